// Decode GEMV family for gfx950: fp16 weights [out, in] row-major, fp32
// accumulation.
//
//  * gemv_f16_kernel   — batch <= 8.  Each wave owns RPW output features and
//    streams their rows once: lane l reads the 16-byte chunks l, l+64, ...
//    (coalesced 1 KiB per wave per load), issues U*RPW chunk loads before
//    any math, accumulates with v_dot2_f32_f16 and reduces the 64 lane
//    partials with DPP row sums + v_readlane.  (Reference: emitDecodeGEMV,
//    DecodeGEMVMetalEmitter.cpp:68-132, one threadgroup per output.)
//  * gate_up_silu_kernel — the same stream over Wg and Wu rows of a feature,
//    finished with the reference's rounding points
//    (emitDecoderGatedMLP, DecoderLLMMetalEmitter.cpp:479-536).
//  * skinny_mfma_kernel — batch >= 9: 16 output features x 16*MT batch rows
//    per block with v_mfma_f32_16x16x32_f16; the block's 4 waves split K in
//    128-element tiles and are summed through LDS.
#include "tmc_abi.hpp"
#include "tmc_device.hpp"

namespace tmc {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

template <int NB, int RPW, int U, typename OutT>
__global__ __launch_bounds__(kThreads) void gemv_f16_kernel(const half_t* __restrict__ x,
                                                           const half_t* __restrict__ w,
                                                           OutT* __restrict__ y, int n_out,
                                                           int k_in) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kWavesPerBlock + wave) * RPW;
  if (row0 >= n_out) return;  // wave-uniform
  const int chunks = k_in >> 3;
  const half_t* wrow[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) wrow[r] = w + (size_t)min(row0 + r, n_out - 1) * k_in;
  float acc[RPW][NB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = 0.0f;

  int c = lane;
  for (; c + kWave * (U - 1) < chunks; c += kWave * U) {
    h8 wv[U][RPW];
    h8 xv[U][NB];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < RPW; ++r) wv[u][r] = load_h8_stream(wrow[r] + 8 * (c + kWave * u));
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int b = 0; b < NB; ++b) xv[u][b] = load_h8(x + (size_t)b * k_in + 8 * (c + kWave * u));
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[r][b] = dot8(wv[u][r], xv[u][b], acc[r][b]);
  }
  for (; c < chunks; c += kWave) {
    h8 xv[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) xv[b] = load_h8(x + (size_t)b * k_in + 8 * c);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const h8 wv = load_h8_stream(wrow[r] + 8 * c);
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][b] = dot8(wv, xv[b], acc[r][b]);
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float total = wave_sum(acc[r][b]);
      if (lane == 0 && row0 + r < n_out) y[(size_t)b * n_out + row0 + r] = from_float<OutT>(total);
    }
}

// Any K (no 16-byte alignment): one wave per (row, feature), scalar loads.
template <typename OutT>
__global__ __launch_bounds__(kThreads) void gemv_f16_generic_kernel(const half_t* __restrict__ x,
                                                                   const half_t* __restrict__ w,
                                                                   OutT* __restrict__ y,
                                                                   int batch, int n_out,
                                                                   int k_in) {
  const int lane = threadIdx.x & (kWave - 1);
  const long item = (long)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (item >= (long)batch * n_out) return;
  const int b = (int)(item / n_out), n = (int)(item % n_out);
  float acc = 0.0f;
  for (int k = lane; k < k_in; k += kWave)
    acc += (float)x[(size_t)b * k_in + k] * (float)w[(size_t)n * k_in + k];
  const float total = wave_sum(acc);
  if (lane == 0) y[(size_t)b * n_out + n] = from_float<OutT>(total);
}

__device__ __forceinline__ half_t silu_mul_h(float gate_sum, float up_sum) {
  const float g = through<half_t>(gate_sum);
  const float u = through<half_t>(up_sum);
  const float activated = through<half_t>(g / (1.0f + expf(-g)));
  return (half_t)(activated * u);
}

template <int NB, int RPW, int U>
__global__ __launch_bounds__(kThreads) void gate_up_silu_kernel(const half_t* __restrict__ x,
                                                               const half_t* __restrict__ wg,
                                                               const half_t* __restrict__ wu,
                                                               half_t* __restrict__ out,
                                                               int inter, int hidden) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kWavesPerBlock + wave) * RPW;
  if (row0 >= inter) return;
  const int chunks = hidden >> 3;
  const half_t* grow[RPW];
  const half_t* urow[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const size_t off = (size_t)min(row0 + r, inter - 1) * hidden;
    grow[r] = wg + off;
    urow[r] = wu + off;
  }
  float ag[RPW][NB], au[RPW][NB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) ag[r][b] = au[r][b] = 0.0f;

  int c = lane;
  for (; c + kWave * (U - 1) < chunks; c += kWave * U) {
    h8 gv[U][RPW], uv[U][RPW], xv[U][NB];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        gv[u][r] = load_h8_stream(grow[r] + 8 * (c + kWave * u));
        uv[u][r] = load_h8_stream(urow[r] + 8 * (c + kWave * u));
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int b = 0; b < NB; ++b) xv[u][b] = load_h8(x + (size_t)b * hidden + 8 * (c + kWave * u));
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          ag[r][b] = dot8(gv[u][r], xv[u][b], ag[r][b]);
          au[r][b] = dot8(uv[u][r], xv[u][b], au[r][b]);
        }
  }
  for (; c < chunks; c += kWave) {
    h8 xv[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) xv[b] = load_h8(x + (size_t)b * hidden + 8 * c);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const h8 gv = load_h8_stream(grow[r] + 8 * c);
      const h8 uv = load_h8_stream(urow[r] + 8 * c);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        ag[r][b] = dot8(gv, xv[b], ag[r][b]);
        au[r][b] = dot8(uv, xv[b], au[r][b]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float g = wave_sum(ag[r][b]);
      const float u = wave_sum(au[r][b]);
      if (lane == 0 && row0 + r < inter) out[(size_t)b * inter + row0 + r] = silu_mul_h(g, u);
    }
}

// Unaligned fallback of the gated MLP: one wave per (row, feature).
__global__ __launch_bounds__(kThreads) void gate_up_silu_generic_kernel(
    const half_t* __restrict__ x, const half_t* __restrict__ wg, const half_t* __restrict__ wu,
    half_t* __restrict__ out, int batch, int inter, int hidden) {
  const int lane = threadIdx.x & (kWave - 1);
  const long item = (long)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (item >= (long)batch * inter) return;
  const int b = (int)(item / inter), f = (int)(item % inter);
  float g = 0.0f, u = 0.0f;
  for (int k = lane; k < hidden; k += kWave) {
    const float xv = (float)x[(size_t)b * hidden + k];
    g += xv * (float)wg[(size_t)f * hidden + k];
    u += xv * (float)wu[(size_t)f * hidden + k];
  }
  const float gs = wave_sum(g), us = wave_sum(u);
  if (lane == 0) out[(size_t)b * inter + f] = silu_mul_h(gs, us);
}

// D[i][j] = sum_k x[i][k] * w[n0+j][k] for MT 16-row tiles of x.  Lane l
// supplies row l%16 of both operands and k-group l/16; within a 128-wide K
// tile group g covers k in [32g, 32g+32), split over 4 MFMAs of 8 k each,
// so each lane reads 64 contiguous bytes per row.  Both operands use the
// same (group, slot) -> k assignment, so the MFMA sum is over exactly the
// tile's k values.
template <int MT, typename OutT>
__global__ __launch_bounds__(kThreads) void skinny_mfma_kernel(const half_t* __restrict__ x,
                                                              const half_t* __restrict__ w,
                                                              OutT* __restrict__ y, int m_rows,
                                                              int n_out, int k_in) {
  __shared__ float partial[kWavesPerBlock][MT][4][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int j = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const half_t* wrow = w + (size_t)min(n0 + j, n_out - 1) * k_in;
  f4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  const int tiles = (k_in + 127) / 128;
  for (int t = wave; t < tiles; t += kWavesPerBlock) {
    const int kb = t * 128 + 32 * g;
    h8 wv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = kb + 8 * s;
      wv[s] = k < k_in ? load_h8_stream(wrow + k) : zero;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = mt * 16 + j;
      h8 xv[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = kb + 8 * s;
        xv[s] = (row < m_rows && k < k_in) ? load_h8(x + (size_t)row * k_in + k) : zero;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[s], wv[s], acc[mt], 0, 0, 0);
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) partial[wave][mt][r][lane] = acc[mt][r];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = (partial[0][mt][r][lane] + partial[1][mt][r][lane]) +
                      (partial[2][mt][r][lane] + partial[3][mt][r][lane]);
      const int row = mt * 16 + 4 * g + r;
      const int col = n0 + j;
      if (row < m_rows && col < n_out) y[(size_t)row * n_out + col] = from_float<OutT>(v);
    }
}

// ---------------------------------------------------------------- dispatch
template <int NB, typename OutT>
int launch_gemv_nb(const half_t* x, const half_t* w, OutT* y, int n, int k, int rpw,
                   hipStream_t stream) {
  constexpr int U = 4;
  const int rows_per_block = kWavesPerBlock * rpw;
  const dim3 grid((n + rows_per_block - 1) / rows_per_block);
  switch (rpw) {
  case 1: hipLaunchKernelGGL((gemv_f16_kernel<NB, 1, U, OutT>), grid, dim3(kThreads), 0, stream, x, w, y, n, k); break;
  case 2: hipLaunchKernelGGL((gemv_f16_kernel<NB, 2, U, OutT>), grid, dim3(kThreads), 0, stream, x, w, y, n, k); break;
  default: hipLaunchKernelGGL((gemv_f16_kernel<NB, 4, U, OutT>), grid, dim3(kThreads), 0, stream, x, w, y, n, k); break;
  }
  return check_launch("gemv_f16_kernel");
}

template <typename OutT>
int launch_gemv(const half_t* x, const half_t* w, OutT* y, int batch, int n, int k, int rpw,
                hipStream_t stream) {
  switch (batch) {
  case 1: return launch_gemv_nb<1>(x, w, y, n, k, rpw, stream);
  case 2: return launch_gemv_nb<2>(x, w, y, n, k, rpw, stream);
  case 3: return launch_gemv_nb<3>(x, w, y, n, k, rpw, stream);
  case 4: return launch_gemv_nb<4>(x, w, y, n, k, rpw, stream);
  case 5: return launch_gemv_nb<5>(x, w, y, n, k, rpw, stream);
  case 6: return launch_gemv_nb<6>(x, w, y, n, k, rpw, stream);
  case 7: return launch_gemv_nb<7>(x, w, y, n, k, rpw, stream);
  default: return launch_gemv_nb<8>(x, w, y, n, k, rpw, stream);
  }
}

template <typename OutT>
int launch_skinny(const half_t* x, const half_t* w, OutT* y, int batch, int n, int k,
                  hipStream_t stream) {
  // 64 batch rows per launch; larger batches re-stream W once per 64 rows.
  for (int r0 = 0; r0 < batch; r0 += 64) {
    const int rows = min(64, batch - r0);
    const dim3 grid((n + 15) / 16);
    const half_t* xs = x + (size_t)r0 * k;
    OutT* ys = y + (size_t)r0 * n;
    switch ((rows + 15) / 16) {
    case 1: hipLaunchKernelGGL((skinny_mfma_kernel<1, OutT>), grid, dim3(kThreads), 0, stream, xs, w, ys, rows, n, k); break;
    case 2: hipLaunchKernelGGL((skinny_mfma_kernel<2, OutT>), grid, dim3(kThreads), 0, stream, xs, w, ys, rows, n, k); break;
    case 3: hipLaunchKernelGGL((skinny_mfma_kernel<3, OutT>), grid, dim3(kThreads), 0, stream, xs, w, ys, rows, n, k); break;
    default: hipLaunchKernelGGL((skinny_mfma_kernel<4, OutT>), grid, dim3(kThreads), 0, stream, xs, w, ys, rows, n, k); break;
    }
    if (check_launch("skinny_mfma_kernel")) return 1;
  }
  return 0;
}

int check_linear_args(const void* x, const void* w, const void* y, int y_dtype, int64_t batch,
                      int64_t k, int64_t n) {
  TMC_REQUIRE(x && w && y, "GEMV: null device pointer.");
  TMC_REQUIRE(y_dtype == TMC_F16 || y_dtype == TMC_F32, "GEMV: output dtype must be fp16 or fp32.");
  TMC_REQUIRE(batch > 0 && k > 0 && n > 0, "GEMV: dimensions must be positive.");
  TMC_REQUIRE(k < (1LL << 31) && n < (1LL << 31) && batch < (1LL << 31),
              "GEMV: dimensions exceed 32-bit indexing.");
  return 0;
}

bool vector_path_ok(const void* x, const void* w, int64_t k) {
  return (k % 8) == 0 && aligned16(x) && aligned16(w);
}

}  // namespace

// Rows per wave for the batch <= 8 path: more rows per wave amortise the x
// loads at larger batch; small N keeps one row per wave for parallelism.
static int choose_rpw(int64_t batch, int64_t n) {
  if (n < 4096) return 1;
  if (batch >= 4) return 2;
  return 1;
}

}  // namespace tmc

using namespace tmc;

extern "C" int tmc_gemv_f16(const void* x, const void* w, void* y, int y_dtype, int64_t batch,
                            int64_t in_features, int64_t out_features, void* stream) {
  if (check_linear_args(x, w, y, y_dtype, batch, in_features, out_features)) return 1;
  if (batch > 8 && vector_path_ok(x, w, in_features))
    return tmc_skinny_gemm_f16_mfma(x, w, y, y_dtype, batch, in_features, out_features, stream);
  const auto* xh = static_cast<const half_t*>(x);
  const auto* wh = static_cast<const half_t*>(w);
  const hipStream_t s = as_stream(stream);
  const int k = (int)in_features, n = (int)out_features;
  if (!vector_path_ok(x, w, in_features)) {
    const long items = (long)batch * n;
    const dim3 grid((unsigned)((items + kWavesPerBlock - 1) / kWavesPerBlock));
    if (y_dtype == TMC_F32)
      hipLaunchKernelGGL((gemv_f16_generic_kernel<float>), grid, dim3(kThreads), 0, s, xh, wh,
                         static_cast<float*>(y), (int)batch, n, k);
    else
      hipLaunchKernelGGL((gemv_f16_generic_kernel<half_t>), grid, dim3(kThreads), 0, s, xh, wh,
                         static_cast<half_t*>(y), (int)batch, n, k);
    return check_launch("gemv_f16_generic_kernel");
  }
  const int rpw = choose_rpw(batch, n);
  for (int64_t r0 = 0; r0 < batch; r0 += 8) {
    const int rows = (int)std::min<int64_t>(8, batch - r0);
    int rc;
    if (y_dtype == TMC_F32)
      rc = launch_gemv<float>(xh + r0 * k, wh, static_cast<float*>(y) + r0 * n, rows, n, k, rpw, s);
    else
      rc = launch_gemv<half_t>(xh + r0 * k, wh, static_cast<half_t*>(y) + r0 * n, rows, n, k, rpw, s);
    if (rc) return rc;
  }
  return 0;
}

extern "C" int tmc_skinny_gemm_f16_mfma(const void* x, const void* w, void* y, int y_dtype,
                                        int64_t batch, int64_t in_features, int64_t out_features,
                                        void* stream) {
  if (check_linear_args(x, w, y, y_dtype, batch, in_features, out_features)) return 1;
  TMC_REQUIRE(vector_path_ok(x, w, in_features),
              "MFMA GEMM: in_features must be a multiple of 8 and x, W 16-byte aligned.");
  const auto* xh = static_cast<const half_t*>(x);
  const auto* wh = static_cast<const half_t*>(w);
  if (y_dtype == TMC_F32)
    return launch_skinny<float>(xh, wh, static_cast<float*>(y), (int)batch, (int)out_features,
                                (int)in_features, as_stream(stream));
  return launch_skinny<half_t>(xh, wh, static_cast<half_t*>(y), (int)batch, (int)out_features,
                               (int)in_features, as_stream(stream));
}

extern "C" int tmc_gate_up_silu_f16(const void* x, const void* w_gate, const void* w_up, void* out,
                                    int64_t batch, int64_t hidden, int64_t intermediate,
                                    void* stream) {
  TMC_REQUIRE(x && w_gate && w_up && out, "Gated MLP: null device pointer.");
  TMC_REQUIRE(batch > 0 && hidden > 0 && intermediate > 0, "Gated MLP: dimensions must be positive.");
  TMC_REQUIRE(hidden < (1LL << 31) && intermediate < (1LL << 31), "Gated MLP: dimensions too large.");
  const auto* xh = static_cast<const half_t*>(x);
  const auto* gh = static_cast<const half_t*>(w_gate);
  const auto* uh = static_cast<const half_t*>(w_up);
  auto* oh = static_cast<half_t*>(out);
  const hipStream_t s = as_stream(stream);
  const int h = (int)hidden, f = (int)intermediate;
  const bool vec = (hidden % 8) == 0 && aligned16(x) && aligned16(w_gate) && aligned16(w_up);
  if (!vec) {
    const long items = (long)batch * f;
    const dim3 grid((unsigned)((items + kWavesPerBlock - 1) / kWavesPerBlock));
    hipLaunchKernelGGL(gate_up_silu_generic_kernel, grid, dim3(kThreads), 0, s, xh, gh, uh, oh,
                       (int)batch, f, h);
    return check_launch("gate_up_silu_generic_kernel");
  }
  constexpr int RPW = 1, U = 4;
  const dim3 grid((f + kWavesPerBlock * RPW - 1) / (kWavesPerBlock * RPW));
  for (int64_t r0 = 0; r0 < batch; r0 += 8) {
    const int rows = (int)std::min<int64_t>(8, batch - r0);
    const half_t* xs = xh + r0 * h;
    half_t* os = oh + r0 * f;
    switch (rows) {
    case 1: hipLaunchKernelGGL((gate_up_silu_kernel<1, RPW, U>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    case 2: hipLaunchKernelGGL((gate_up_silu_kernel<2, RPW, U>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    case 3: hipLaunchKernelGGL((gate_up_silu_kernel<3, RPW, U>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    case 4: hipLaunchKernelGGL((gate_up_silu_kernel<4, RPW, U>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    case 5: hipLaunchKernelGGL((gate_up_silu_kernel<5, RPW, 2>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    case 6: hipLaunchKernelGGL((gate_up_silu_kernel<6, RPW, 2>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    case 7: hipLaunchKernelGGL((gate_up_silu_kernel<7, RPW, 2>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    default: hipLaunchKernelGGL((gate_up_silu_kernel<8, RPW, 2>), grid, dim3(kThreads), 0, s, xs, gh, uh, os, f, h); break;
    }
    if (check_launch("gate_up_silu_kernel")) return 1;
  }
  return 0;
}
