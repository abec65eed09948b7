// Decode GEMV family for gfx950: fp16 weights [out, in] row-major, fp32
// accumulation.  Two algorithms, both streaming every weight byte once:
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
// The gated MLP (emitDecoderGatedMLP, DecoderLLMMetalEmitter.cpp:479-536)
// runs either algorithm over the Wg and Wu rows of each feature and finishes
// with the reference rounding points h(h(silu(h(g))) * h(u)).
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
template <int MATS, int NB, int RPW, int U, int KS, typename OutT>
__global__ __launch_bounds__(256) void gemv_dot_kernel(const half_t* __restrict__ x,
                                                      const half_t* __restrict__ w0,
                                                      const half_t* __restrict__ w1,
                                                      OutT* __restrict__ y, int n_out, int k_in) {
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
        const h8 wv = load_h8_stream(wrow[m][r] + 8 * c);
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[m][r][b] = dot8(wv, xv[b], acc[m][r][b]);
      }
  }
  if constexpr (KS == 1) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float a0 = wave_sum(acc[0][r][b]);
        const float a1 = MATS == 2 ? wave_sum(acc[MATS - 1][r][b]) : 0.0f;
        if (lane == 0 && live && row0 + r < n_out)
          write_out<MATS>(y, (size_t)b * n_out + row0 + r, a0, a1);
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
    if (part == 0 && live) {
      for (int idx = lane; idx < RPW * NB; idx += kWave) {
        const int r = idx / NB, b = idx % NB;
        float a[2] = {0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
          for (int s = 0; s < KS; ++s) a[m] += partial[wave + s][m][r][b];
        if (row0 + r < n_out) write_out<MATS>(y, (size_t)b * n_out + row0 + r, a[0], a[1]);
      }
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

// ---------------------------------------------------------------- dispatch
struct Shape {
  const half_t* x;
  const half_t* w0;
  const half_t* w1;
  void* y;
  int y_dtype, batch, n, k;
};

template <int MATS, int NB, int RPW, int U, int KS, typename OutT>
int launch_dot(const Shape& s, const half_t* x, OutT* y, hipStream_t stream) {
  const int rows_per_block = (4 / KS) * RPW;
  const dim3 grid((s.n + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL((gemv_dot_kernel<MATS, NB, RPW, U, KS, OutT>), grid, dim3(256), 0, stream, x,
                     s.w0, s.w1, y, s.n, s.k);
  return check_launch("gemv_dot_kernel");
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

// Default configuration per shape (the tuner may override it), from graph-
// timed sweeps on MI355X: batch 1 streams rows with the dot algorithm and 4
// waves per row (2 rows per wave for rows longer than 8K); larger batches use
// MFMA with one 16-row tile per block, 2 waves per tile for the gated pair
// and 16 for a single matrix.
tmc_gemv_config default_config(int batch, int n, int k, int mats) {
  tmc_gemv_config c{};
  (void)n;
  if (batch == 1) {
    c.algorithm = 1;
    c.rows_per_wave = k > 8192 ? 2 : 1;
    c.unroll = mats == 2 ? 2 : 4;
    c.k_split = 4;
  } else {
    c.algorithm = 2;
    c.rows_per_wave = 1;
    c.unroll = 2;
    c.k_split = mats == 2 ? 2 : 16;
    const int tiles = (k + 127) / 128;
    while (c.k_split > 1 && tiles < 2 * c.k_split) c.k_split /= 2;
  }
  return c;
}

int validate_config(const tmc_gemv_config& c) {
  if (c.algorithm == 1) {
    TMC_REQUIRE((c.rows_per_wave == 1 || c.rows_per_wave == 2) &&
                    (c.unroll == 2 || c.unroll == 4) &&
                    (c.k_split == 1 || c.k_split == 2 || c.k_split == 4),
                "GEMV config: dot algorithm needs rows_per_wave 1|2, unroll 2|4, k_split 1|2|4.");
  } else if (c.algorithm == 2) {
    TMC_REQUIRE(c.rows_per_wave >= 1 && c.k_split >= 1 && c.rows_per_wave * c.k_split <= 16 &&
                    (c.unroll == 1 || c.unroll == 2),
                "GEMV config: MFMA needs n_tiles * k_split <= 16 waves and unroll 1|2.");
  } else {
    return fail("GEMV config: algorithm must be 0 (auto), 1 (dot) or 2 (MFMA).");
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
  if (cfg.algorithm == 1) {
    if (mats == 2) return run_dot<2, half_t>(s, cfg, st);
    return y_dtype == TMC_F32 ? run_dot<1, float>(s, cfg, st) : run_dot<1, half_t>(s, cfg, st);
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
  tmc_gemv_config cfg = default_config(2, (int)out_features, (int)in_features, 1);
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

extern "C" int tmc_gemv_default_config(int64_t batch, int64_t in_features, int64_t out_features,
                                       int gated, tmc_gemv_config* out) {
  TMC_REQUIRE(out && batch > 0 && in_features > 0 && out_features > 0,
              "tmc_gemv_default_config: invalid arguments.");
  *out = default_config((int)batch, (int)out_features, (int)in_features, gated ? 2 : 1);
  return 0;
}
