// Skinny GEMM over fragment-packed fp16 weights (batch > 1 decode) for
// gfx950.  Same arithmetic as the decode GEMV / gated MLP (emitDecodeGEMV,
// DecodeGEMVMetalEmitter.cpp:68-132; emitDecoderGatedMLP,
// DecoderLLMMetalEmitter.cpp:479-536): y[r,n] = sum_k x[r,k] W[n,k], fp32
// accumulation; only the weight layout in HBM differs.
//
// Packed layout.  W [N, K] row-major becomes tiles of 16 output rows x 32 k:
// tile (nt, c) holds rows 16nt..16nt+15 and k 32c..32c+31 as 64 lanes x 8
// halves, lane l = (n % 16) + 16 * ((k % 32) / 8), element k % 8 -- exactly
// the B operand of v_mfma_f32_16x16x32_f16 -- stored at
// ((nt * C + c) * 64 + l) * 16 bytes, C = ceil(K / 32); rows past N and k
// past K are zero.  One weight load instruction of a wave then reads 1 KiB of
// contiguous HBM (a row-major fragment touches 16 rows K*2 bytes apart), which
// measured 20-25% faster for 16-row activations on MI355X.
//
// Kernel: one block per 16-row output tile; KS waves split the K tiles of
// 128 (4 fragments) into contiguous runs, U tiles in flight per wave, and meet
// in LDS.  Activations stay row-major; batch rows past B and k past K read
// as zero through buffer-load range checks.
#include "tmc_abi.hpp"
#include "tmc_device.hpp"

namespace tmc {
namespace {

constexpr unsigned kNone = 0xFFFFFFF0u;  // buffer offset that reads as zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ h8 buffer_load16(__amdgpu_buffer_rsrc_t r, unsigned offset) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)offset, 0, 0));
}
// Weight fragments are read once per launch: non-temporal hint (cache policy
// bit nt), so that they do not evict the activation fragments every output
// tile re-reads from L2.  Measured on MI355X against the default policy:
// C2 at batch 8 5.22 -> 5.60 TB/s, the 7B decode step at batch 16 4706 ->
// 4897 tokens/s.
__device__ __forceinline__ h8 buffer_load16_stream(__amdgpu_buffer_rsrc_t r, unsigned offset) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)offset, 0, 2));
}

__device__ __forceinline__ half_t gated_value(float gate_sum, float up_sum) {
  // h(h(silu(h(g))) * h(u)), DecoderLLMMetalEmitter.cpp:528-532
  const float g = through<half_t>(gate_sum);
  const float u = through<half_t>(up_sum);
  const float activated = through<half_t>(g / (1.0f + expf(-g)));
  return (half_t)(activated * u);
}

// One thread per packed lane slot (16 bytes).  gamma (may be null): the
// slot holds fp16(W[row, k] * gamma[k]), the weights of a projection with
// the preceding RMSNorm's gamma folded in.
__global__ __launch_bounds__(256) void pack_kernel(const half_t* __restrict__ w,
                                                   const half_t* __restrict__ gamma,
                                                   half_t* __restrict__ packed, int n, int k,
                                                   long slots) {
  const int chunks = (k + 31) / 32;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < slots;
       i += (long)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    const long frag = i >> 6;
    const int c = (int)(frag % chunks);
    const int nt = (int)(frag / chunks);
    const int row = nt * 16 + (lane & 15);
    const int k0 = c * 32 + 8 * (lane >> 4);
    h8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = (row < n && k0 + e < k) ? w[(size_t)row * k + k0 + e] : (half_t)0.0f;
      if (gamma && k0 + e < k) v[e] = (half_t)((float)v[e] * (float)gamma[k0 + e]);
    }
    *reinterpret_cast<h8*>(packed + i * 8) = v;
  }
}

// Folded neighbours of a packed GEMM (batch > 1 decode, no norm launch):
//  kPackedNorm: RMSNorm (emitDecoderRMSNorm, DecoderLLMMetalEmitter.cpp:
//    63-108) folded into the projection, as the reference's fusion candidate
//    emitDecoderQKVFusion (:538-602) folds it: x is the residual stream s,
//    the packed weights hold W . diag(gamma) (pack_kernel with gamma), and
//    each output row r is scaled by 1 / sqrt(sum_k s[r, k]^2 / K + eps), the
//    squares taken from the activation fragments the MFMA reads.  The fp16
//    rounding falls on W * gamma rather than on the normalized value.  (A
//    gamma fragment loaded beside every activation fragment measured 1.9 us
//    slower on the batch-16 q.k.v projection: activation-side loads are what
//    these kernels are sensitive to.)
//  kPackedResidual: y = fp16(fp16(acc) + residual), residual in y's layout
//    (emitLinearResidual, :604-621).
enum PackedFuse : int { kPackedPlain = 0, kPackedNorm = 1, kPackedResidual = 2 };

struct PackedFuseArgs {
  const half_t* residual = nullptr;  // kPackedResidual: this pass, in y's layout
  float eps = 0.0f;                  // kPackedNorm
  int argmax_rows = 0;               // ARGMAX: rows of the partial-argmax workspace
};

// XP: x is one 16-row pass in fragment order (lane l of chunk c holds row
// l % 16, k 32c + 8(l / 16) .. +7, the A operand as loaded); YP: the fp16
// output pass is written in the same order for the next GEMM.
// ROPE: y is not written; the q.k.v projection's column pairs of each batch
// row go through rope_append_pair (RoPE + paged append, request
// ra.request_base + row).
// At most kPackedNormWaves waves per tile with the folded norm (its extra
// registers fit the 256-thread bound; the q.k.v, gated and LM head
// defaults use 1-4).
constexpr int kPackedNormWaves = 4;

// ARGMAX (the token-only LM head, emitLMHeadPartialArgmax,
// DecoderLLMMetalEmitter.cpp:700-728): y is a partial-argmax workspace
// (argmax_partials, pf.argmax_rows rows of n_out slots); the tile writes,
// for each batch row, the greatest (value, column) of its 16 logits in the
// greedy-token order to slot blockIdx.x of that row, and block 0 writes the
// slot count.  The values are the logits the plain form stores.
template <int MATS, int U, typename OutT, bool XP = false, bool YP = false, bool ROPE = false,
          int FUSE = kPackedPlain, bool ARGMAX = false>
__global__ __launch_bounds__(FUSE == kPackedNorm ? kPackedNormWaves * kWave : 1024) void packed_gemm_kernel(const half_t* __restrict__ x,
                                                           const half_t* __restrict__ p0,
                                                           const half_t* __restrict__ p1,
                                                           OutT* __restrict__ y, int m_rows,
                                                           int n_out, int k_in, int ks_count,
                                                           unsigned packed_bytes, RopeArgs ra,
                                                           PackedFuseArgs pf) {
  static_assert(!ROPE || (MATS == 1 && !YP), "the RoPE epilogue serves the q.k.v projection");
  static_assert(FUSE != kPackedResidual || (MATS == 1 && !ROPE), "residual: plain projection");
  static_assert(!ARGMAX || (MATS == 1 && !ROPE && !YP && FUSE != kPackedResidual),
                "the argmax epilogue follows one fp32 projection");
  extern __shared__ float red[];  // [ks][MATS][4][64], then kPackedNorm: [ks][16] squares
  const int lane = threadIdx.x & (kWave - 1);
  const int ks = threadIdx.x / kWave;
  const int j = lane & 15;
  const int g = lane >> 4;
  const int nt = blockIdx.x;
  const int chunks = (k_in + 31) / 32;
  const __amdgpu_buffer_rsrc_t rx =
      buffer_rsrc(x, XP ? (unsigned)chunks * 1024u : (unsigned)m_rows * (unsigned)k_in * 2u);
  const __amdgpu_buffer_rsrc_t r0 = buffer_rsrc(p0, packed_bytes);
  const __amdgpu_buffer_rsrc_t r1 = buffer_rsrc(MATS == 2 ? p1 : p0, packed_bytes);
  const unsigned x_row = j < m_rows ? (unsigned)j * (unsigned)k_in * 2u : kNone;
  const unsigned w_base = (unsigned)nt * (unsigned)chunks * 1024u + (unsigned)lane * 16u;
  // Output element of epilogue item q of this thread (item = threadIdx.x +
  // q * threads, < 4 * 64): (row, col) and its index in y's layout.
  auto item_at = [&](int idx, int& row, int& col) -> size_t {
    const int l = idx % kWave, r = idx / kWave;
    row = 4 * (l >> 4) + r;
    col = nt * 16 + (l & 15);
    if constexpr (YP)  // pass-relative fragment slot of (row, col)
      return ((size_t)(col >> 5) * 64 + row + 16 * ((col & 31) >> 3)) * 8 + (col & 7);
    return (size_t)row * n_out + col;
  };
  // kPackedResidual: the residual of each epilogue item is loaded first, ahead
  // of the weight stream, so the epilogue waits on no memory (at batch 16 the
  // o and down projections run one block per CU and end together, so a load
  // in the epilogue was a round trip at the end of every launch)
  constexpr int kItems = 4;  // epilogue items per thread at one wave per tile
  half_t res_pre[kItems];
  if constexpr (FUSE == kPackedResidual) {
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int idx = (int)threadIdx.x + q * ks_count * kWave;
      int row, col;
      const size_t at = item_at(idx < 4 * kWave ? idx : 0, row, col);
      res_pre[q] = idx < 4 * kWave && row < m_rows && col < n_out ? pf.residual[at] : half_t(0.0f);
    }
  }
  float squares = 0.0f;  // kPackedNorm: row j's sum of squares over this lane's k
  f4 acc[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) acc[m] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const int tiles = (chunks + 3) / 4;
  const int per_wave = (tiles + ks_count - 1) / ks_count;
  const int first = ks * per_wave;
  const int last = min(tiles, first + per_wave);
  for (int t0 = first; t0 < last; t0 += U) {
    h8 xv[U][4], wv[U][MATS][4];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int c = (t0 + u) * 4 + s;
        const bool live = t0 + u < last && c < chunks;
        const unsigned w_off = live ? w_base + (unsigned)c * 1024u : kNone;
        wv[u][0][s] = buffer_load16_stream(r0, w_off);
        if constexpr (MATS == 2) wv[u][1][s] = buffer_load16_stream(r1, w_off);
        const int kk = c * 32 + 8 * g;
        if constexpr (XP)  // rows past the batch are never read (their slots are unset)
          xv[u][s] = buffer_load16(
              rx, live && kk < k_in && j < m_rows ? ((unsigned)c * 64u + (unsigned)lane) * 16u
                                                  : kNone);
        else
          xv[u][s] = buffer_load16(
              rx, live && kk < k_in && x_row != kNone ? x_row + (unsigned)kk * 2u : kNone);
      }
    if constexpr (FUSE == kPackedNorm) {
      // every load of the step goes out before the squares (left to itself
      // the scheduler interleaves them and waits after every few)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int s = 0; s < 4; ++s) squares = dot8(xv[u][s], xv[u][s], squares);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int m = 0; m < MATS; ++m)
          acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[u][s], wv[u][m][s], acc[m], 0, 0, 0);
  }
  float* red_sq = red + ks_count * MATS * 4 * kWave;
  if constexpr (FUSE == kPackedNorm) {
    squares += __shfl_xor(squares, 16, kWave);
    squares += __shfl_xor(squares, 32, kWave);
    if (g == 0) red_sq[ks * 16 + j] = squares;
  }
  // kPackedNorm: 1 / rms of batch row `row` (its waves' squares in order)
  auto row_scale = [&](int row) -> float {
    if constexpr (FUSE != kPackedNorm) {
      return 1.0f;
    } else {
      float total = 0.0f;
      for (int w = 0; w < ks_count; ++w) total += red_sq[w * 16 + row];
      return 1.0f / sqrtf(total / (float)k_in + pf.eps);
    }
  };
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((ks * MATS + m) * 4 + r) * kWave + lane] = acc[m][r];
  __syncthreads();
  if constexpr (ROPE) {
    // 16 batch rows x 8 column pairs of the tile; the pair's even column sits
    // in lane 16g + 2p and the odd one in the next lane
    for (int idx = threadIdx.x; idx < 128; idx += ks_count * kWave) {
      const int p = idx & 7, row = idx >> 3;
      const int l = 16 * (row >> 2) + 2 * p, r = row & 3;
      float even = 0.0f, odd = 0.0f;
      for (int w = 0; w < ks_count; ++w) {
        even += red[(w * 4 + r) * kWave + l];
        odd += red[(w * 4 + r) * kWave + l + 1];
      }
      const int col = nt * 16 + 2 * p;
      const float scale = row_scale(row);
      if (row < m_rows && col < n_out)
        rope_append_pair(ra, ra.request_base + row, col, even * scale, odd * scale);
    }
    return;
  }
  if constexpr (ARGMAX) {
    __shared__ float arg_v[16][16];
    __shared__ int arg_i[16][16];
    for (int idx = threadIdx.x; idx < 4 * kWave; idx += ks_count * kWave) {
      const int l = idx % kWave, r = idx / kWave;
      float a = 0.0f;
      for (int w = 0; w < ks_count; ++w) a += red[(w * 4 + r) * kWave + l];
      const int row = 4 * (l >> 4) + r;
      const int col = nt * 16 + (l & 15);
      arg_v[row][l & 15] = col < n_out ? from_float<OutT>(a * row_scale(row)) : -INFINITY;
      arg_i[row][l & 15] = col < n_out ? col : -1;
    }
    __syncthreads();
    if ((int)threadIdx.x < 16 && (int)threadIdx.x < m_rows) {
      const int row = threadIdx.x;
      float best = -INFINITY;
      int selected = -1;
      for (int c = 0; c < 16; ++c)
        if (argmax_better(arg_v[row][c], arg_i[row][c], best, selected)) {
          best = arg_v[row][c];
          selected = arg_i[row][c];
        }
      const ArgmaxPartials out = argmax_partials(y, pf.argmax_rows, n_out);
      const size_t at = (size_t)(ra.request_base + row) * n_out + blockIdx.x;
      out.values[at] = best;
      out.indices[at] = selected;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && ra.request_base == 0) {
      const ArgmaxPartials out = argmax_partials(y, pf.argmax_rows, n_out);
      *out.count = (int)gridDim.x;
    }
    return;
  }
  // acc[r] of lane (j, g) = out[batch 4g + r][row 16nt + j]
#pragma unroll
  for (int q = 0; q < kItems; ++q) {
    const int idx = (int)threadIdx.x + q * ks_count * kWave;
    if (idx >= 4 * kWave) break;
    const int l = idx % kWave, r = idx / kWave;
    float a[2] = {0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < MATS; ++m)
      for (int w = 0; w < ks_count; ++w) a[m] += red[((w * MATS + m) * 4 + r) * kWave + l];
    int row, col;
    const size_t at = item_at(idx, row, col);
    if (row < m_rows && col < n_out) {
      const float scale = row_scale(row);
      if constexpr (MATS == 2)
        y[at] = gated_value(a[0] * scale, a[1] * scale);
      else if constexpr (FUSE == kPackedResidual)
        y[at] = from_float<OutT>(to_float<half_t>(res_pre[q]) +
                                 to_float<half_t>(from_float<half_t>(a[0])));
      else
        y[at] = from_float<OutT>(a[0] * scale);
    }
  }
}

int64_t packed_elements(int64_t n, int64_t k) { return ((n + 15) / 16) * 16 * ((k + 31) / 32) * 32; }

// Default (unroll, k_split) per shape from MI355X sweeps at batch 8 and 16
// with weights beyond the Infinity Cache (K 4096 unless noted): N 32000 ->
// 1 wave per tile; the gated N 11008 pair -> 4 waves (batch 16: 32.9 us
// against 34.4 with 1); N 12288 -> 2 waves (4 at batch 8); N 4096 (K 4096
// and 11008) -> 16 waves from batch 8 (o 7.9 against 8.2 us, down 16.0
// against 16.4 at batch 16), 8 below.  Wide N streams with few waves per
// tile; narrow N needs more waves per tile to fill 256 CUs.  (Sharing each
// activation fragment across 2 or 4 output tiles per block measured slower
// at batch 16: the activation loads do not bound these kernels.)
void default_packed(int64_t batch, int64_t n, int mats, int& unroll, int& ks) {
  unroll = 2;
  if (mats == 2)
    ks = 4;
  else if (n >= 16384)
    ks = 1;
  else if (n >= 8192)
    ks = batch > 8 ? 2 : 4;
  else
    ks = batch >= 8 ? 16 : 8;
}

// K tiles in flight per wave of the norm-folded LM head (N >= 16384, one
// wave per 16-column tile), from MI355X sweeps at N 32000, K 4096 with
// rotating weights: batch 16 1 (41.9 us against 44.8 with 2), batches 2-8 4
// (40.3-40.8 against 40.8-41.4 us).  The norm form's 256-thread bound leaves
// 4 tiles in flight without spills.
int lm_head_unroll(int64_t batch) { return batch > 8 ? 1 : 4; }

template <int MATS, typename OutT, bool XP, bool YP, bool ROPE = false, int FUSE = kPackedPlain,
          bool ARGMAX = false>
int run_packed(const half_t* x, const half_t* p0, const half_t* p1, OutT* y, int64_t batch,
               int64_t k, int64_t n, int unroll, int ks, hipStream_t st,
               const RopeArgs& rope = RopeArgs{}, const PackedFuseArgs& fuse = PackedFuseArgs{}) {
  const int64_t bytes = packed_elements(n, k) * 2;
  const dim3 grid((unsigned)((n + 15) / 16));
  const size_t lds = (size_t)ks * MATS * 4 * kWave * sizeof(float) +
                     (FUSE == kPackedNorm ? (size_t)ks * 16 * sizeof(float) : 0);
  const int64_t x_pass = XP ? ((k + 31) / 32) * 512 : 16 * k;  // elements per 16-row pass
  const int64_t y_pass = YP ? ((n + 31) / 32) * 512 : 16 * n;
  for (int64_t r0 = 0; r0 < batch; r0 += 16) {
    const int rows = (int)std::min<int64_t>(16, batch - r0);
    const half_t* xs = x + (r0 / 16) * x_pass;
    OutT* ys = ROPE || ARGMAX ? y : y + (r0 / 16) * y_pass;
    RopeArgs ra = rope;
    ra.request_base = (int)r0;
    PackedFuseArgs pf = fuse;
    if (FUSE == kPackedResidual) pf.residual = fuse.residual + (r0 / 16) * y_pass;
    if (unroll == 1)
      hipLaunchKernelGGL((packed_gemm_kernel<MATS, 1, OutT, XP, YP, ROPE, FUSE, ARGMAX>), grid,
                         dim3(ks * kWave), lds, st, xs, p0, p1, ys, rows, (int)n, (int)k, ks,
                         (unsigned)bytes, ra, pf);
    else if (unroll == 2)
      hipLaunchKernelGGL((packed_gemm_kernel<MATS, 2, OutT, XP, YP, ROPE, FUSE, ARGMAX>), grid,
                         dim3(ks * kWave), lds, st, xs, p0, p1, ys, rows, (int)n, (int)k, ks,
                         (unsigned)bytes, ra, pf);
    else
      hipLaunchKernelGGL((packed_gemm_kernel<MATS, 4, OutT, XP, YP, ROPE, FUSE, ARGMAX>), grid,
                         dim3(ks * kWave), lds, st, xs, p0, p1, ys, rows, (int)n, (int)k, ks,
                         (unsigned)bytes, ra, pf);
    if (check_launch("packed_gemm_kernel")) return 1;
  }
  return 0;
}

template <int MATS, typename OutT, int FUSE = kPackedPlain>
int run_packed_layout(const half_t* x, const half_t* p0, const half_t* p1, OutT* y,
                      int64_t batch, int64_t k, int64_t n, int unroll, int ks, int layout,
                      hipStream_t st, const PackedFuseArgs& pf = PackedFuseArgs{}) {
  const bool xp = layout & TMC_LAYOUT_X_PACKED, yp = layout & TMC_LAYOUT_Y_PACKED;
  const RopeArgs none{};
  if (xp && yp)
    return run_packed<MATS, OutT, true, true, false, FUSE>(x, p0, p1, y, batch, k, n, unroll, ks,
                                                           st, none, pf);
  if (xp)
    return run_packed<MATS, OutT, true, false, false, FUSE>(x, p0, p1, y, batch, k, n, unroll, ks,
                                                            st, none, pf);
  if (yp)
    return run_packed<MATS, OutT, false, true, false, FUSE>(x, p0, p1, y, batch, k, n, unroll, ks,
                                                            st, none, pf);
  return run_packed<MATS, OutT, false, false, false, FUSE>(x, p0, p1, y, batch, k, n, unroll, ks,
                                                           st, none, pf);
}

// One thread per 8-element slot of a 16-row pass in fragment order.
__global__ __launch_bounds__(256) void pack_activations_kernel(const half_t* __restrict__ src,
                                                               half_t* __restrict__ dst, int rows,
                                                               int cols, int unpack, long slots) {
  const int chunks = (cols + 31) / 32;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < slots;
       i += (long)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    const long frag = i >> 6;
    const int c = (int)(frag % chunks);
    const long pass = frag / chunks;
    const long row = pass * 16 + (lane & 15);
    const int col = c * 32 + 8 * (lane >> 4);
    if (row >= rows || col >= cols) continue;
    const size_t rm = (size_t)row * cols + col;
    if (unpack)
      *reinterpret_cast<h8*>(dst + rm) = *reinterpret_cast<const h8*>(src + i * 8);
    else
      *reinterpret_cast<h8*>(dst + i * 8) = *reinterpret_cast<const h8*>(src + rm);
  }
}

int packed_entry(int mats, const void* x, const void* p0, const void* p1, void* y, int y_dtype,
                 int64_t batch, int64_t k, int64_t n, int layout, const tmc_gemv_config* config,
                 void* stream, int fuse = kPackedPlain, const PackedFuseArgs& pf = PackedFuseArgs{}) {
  const char* what = mats == 2 ? "Packed gated MLP" : "Packed GEMM";
  TMC_REQUIRE(fuse != kPackedNorm || (pf.eps > 0.0f && std::isfinite(pf.eps)),
              std::string(what) + " with RMSNorm: epsilon must be positive.");
  TMC_REQUIRE(fuse != kPackedResidual || (mats == 1 && y_dtype == TMC_F16 && pf.residual),
              std::string(what) + " with residual: fp16 output and a residual are required.");
  TMC_REQUIRE(x && p0 && y && (mats == 1 || p1), std::string(what) + ": null device pointer.");
  TMC_REQUIRE(y_dtype == TMC_F16 || y_dtype == TMC_F32,
              std::string(what) + ": output dtype must be fp16 or fp32.");
  TMC_REQUIRE(batch > 0 && k > 0 && n > 0, std::string(what) + ": dimensions must be positive.");
  TMC_REQUIRE(k % 8 == 0 && aligned16(x) && aligned16(p0) && (mats == 1 || aligned16(p1)),
              std::string(what) + ": in_features must be a multiple of 8 and x, W 16-byte aligned.");
  TMC_REQUIRE((uint64_t)packed_elements(n, k) * 2 < kNone && (uint64_t)16 * k * 2 < kNone &&
                  n < (1LL << 31) && batch < (1LL << 31),
              std::string(what) + ": operands exceed the 4 GiB buffer range.");
  int unroll, ks;
  default_packed(batch, n, mats, unroll, ks);
  // folded norm: 4 waves per tile below the LM head's width (batch 16 q.k.v
  // 20.5-20.9 us against 21.5 with the plain default of 2)
  if (fuse == kPackedNorm) ks = n >= 16384 ? std::min(ks, kPackedNormWaves) : kPackedNormWaves;
  if (fuse == kPackedNorm && n >= 16384) unroll = lm_head_unroll(batch);
  if (config && config->algorithm != 0) {
    unroll = config->unroll;
    ks = config->k_split;
  }
  TMC_REQUIRE((unroll == 1 || unroll == 2 || unroll == 4) && ks >= 1 &&
                  ks <= (fuse == kPackedNorm ? kPackedNormWaves : 16),
              std::string(what) + ": config needs unroll 1|2|4 and k_split 1..16 (1..4 with "
              "RMSNorm).");
  TMC_REQUIRE((layout & ~(TMC_LAYOUT_X_PACKED | TMC_LAYOUT_Y_PACKED)) == 0,
              std::string(what) + ": unknown layout bits.");
  TMC_REQUIRE(!(layout & TMC_LAYOUT_Y_PACKED) || y_dtype == TMC_F16,
              std::string(what) + ": a packed output must be fp16.");
  TMC_REQUIRE(!(layout & TMC_LAYOUT_Y_PACKED) || aligned16(y),
              std::string(what) + ": a packed output must be 16-byte aligned.");
  const hipStream_t st = as_stream(stream);
  const half_t* xs = static_cast<const half_t*>(x);
  const half_t* a = static_cast<const half_t*>(p0);
  const half_t* b = static_cast<const half_t*>(p1);
  if (fuse == kPackedNorm) {
    if (mats == 2)
      return run_packed_layout<2, half_t, kPackedNorm>(xs, a, b, static_cast<half_t*>(y), batch, k,
                                                       n, unroll, ks, layout, st, pf);
    if (y_dtype == TMC_F32)
      return run_packed_layout<1, float, kPackedNorm>(xs, a, a, static_cast<float*>(y), batch, k,
                                                      n, unroll, ks, layout & TMC_LAYOUT_X_PACKED,
                                                      st, pf);
    return run_packed_layout<1, half_t, kPackedNorm>(xs, a, a, static_cast<half_t*>(y), batch, k,
                                                     n, unroll, ks, layout, st, pf);
  }
  if (fuse == kPackedResidual)
    return run_packed_layout<1, half_t, kPackedResidual>(xs, a, a, static_cast<half_t*>(y), batch,
                                                         k, n, unroll, ks, layout, st, pf);
  if (mats == 2)
    return run_packed_layout<2, half_t>(xs, a, b, static_cast<half_t*>(y), batch, k, n, unroll,
                                        ks, layout, st);
  if (y_dtype == TMC_F32)
    return run_packed_layout<1, float>(xs, a, a, static_cast<float*>(y), batch, k, n, unroll, ks,
                                       layout & TMC_LAYOUT_X_PACKED, st);
  return run_packed_layout<1, half_t>(xs, a, a, static_cast<half_t*>(y), batch, k, n, unroll, ks,
                                      layout, st);
}

}  // namespace
}  // namespace tmc

using namespace tmc;

extern "C" int64_t tmc_packed_weight_elements(int64_t out_features, int64_t in_features) {
  if (out_features <= 0 || in_features <= 0) return 0;
  return packed_elements(out_features, in_features);
}

extern "C" int tmc_pack_weights_scaled_f16(const void* w, const void* gamma, void* packed,
                                           int64_t out_features, int64_t in_features,
                                           void* stream) {
  TMC_REQUIRE(w && packed, "Pack weights: null device pointer.");
  TMC_REQUIRE(out_features > 0 && in_features > 0 && out_features < (1LL << 31) &&
                  in_features < (1LL << 31),
              "Pack weights: invalid shape.");
  TMC_REQUIRE(aligned16(packed), "Pack weights: the packed buffer must be 16-byte aligned.");
  const long slots = (long)(packed_elements(out_features, in_features) / 8);
  const unsigned blocks = (unsigned)std::min<long>((slots + 255) / 256, 65536);
  hipLaunchKernelGGL(pack_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                     static_cast<const half_t*>(w), static_cast<const half_t*>(gamma),
                     static_cast<half_t*>(packed), (int)out_features, (int)in_features, slots);
  return check_launch("pack_kernel");
}

extern "C" int tmc_pack_weights_f16(const void* w, void* packed, int64_t out_features,
                                    int64_t in_features, void* stream) {
  return tmc_pack_weights_scaled_f16(w, nullptr, packed, out_features, in_features, stream);
}

extern "C" int tmc_gemm_packed_f16(const void* x, const void* packed_w, void* y, int y_dtype,
                                   int64_t batch, int64_t in_features, int64_t out_features,
                                   const tmc_gemv_config* config, void* stream) {
  return packed_entry(1, x, packed_w, nullptr, y, y_dtype, batch, in_features, out_features, 0,
                      config, stream);
}

extern "C" int tmc_gate_up_silu_packed_f16(const void* x, const void* packed_gate,
                                           const void* packed_up, void* out, int64_t batch,
                                           int64_t hidden, int64_t intermediate,
                                           const tmc_gemv_config* config, void* stream) {
  return packed_entry(2, x, packed_gate, packed_up, out, TMC_F16, batch, hidden, intermediate, 0,
                      config, stream);
}

extern "C" int tmc_gemm_packed_ex_f16(const void* x, const void* packed_w, void* y, int y_dtype,
                                      int64_t batch, int64_t in_features, int64_t out_features,
                                      int layout, const tmc_gemv_config* config, void* stream) {
  return packed_entry(1, x, packed_w, nullptr, y, y_dtype, batch, in_features, out_features,
                      layout, config, stream);
}

namespace tmc {
namespace {

int qkv_rope_packed_entry(const void* x, bool norm, float eps, const void* packed_w,
                          const float* cosine, const float* sine, const int32_t* valid_lengths,
                          const int32_t* block_tables, const int32_t* active_count, void* q_out,
                          void* key_pool, void* value_pool, int64_t batch, int64_t hidden,
                          int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t capacity,
                          int64_t page_size, int64_t max_pages, int layout,
                          const tmc_gemv_config* config, void* stream) {
  TMC_REQUIRE(x && packed_w && cosine && sine && valid_lengths && block_tables && active_count &&
                  q_out && key_pool && value_pool,
              "Packed q.k.v RoPE append: null pointer.");
  TMC_REQUIRE(!norm || (eps > 0.0f && std::isfinite(eps)),
              "Packed q.k.v RoPE append with RMSNorm: epsilon must be positive.");
  TMC_REQUIRE(batch > 0 && batch < (1LL << 31) && hidden > 0 && hidden % 8 == 0 &&
                  aligned16(x) && aligned16(packed_w),
              "Packed q.k.v RoPE append: hidden must be a positive multiple of 8 and x, W "
              "16-byte aligned.");
  TMC_REQUIRE(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 && head_dim > 0 &&
                  head_dim % 2 == 0 && capacity > 0 && capacity < (1LL << 31) && page_size > 0 &&
                  page_size <= capacity && max_pages == (capacity + page_size - 1) / page_size &&
                  (q_heads + 2 * kv_heads) * head_dim < (1LL << 31),
              "Packed q.k.v RoPE append: invalid head geometry or capacity (max_pages must be "
              "ceil(capacity / page_size)).");
  const int64_t n = (q_heads + 2 * kv_heads) * head_dim;
  TMC_REQUIRE((uint64_t)packed_elements(n, hidden) * 2 < kNone && (uint64_t)16 * hidden * 2 < kNone,
              "Packed q.k.v RoPE append: operands exceed the 4 GiB buffer range.");
  TMC_REQUIRE((layout & ~TMC_LAYOUT_X_PACKED) == 0,
              "Packed q.k.v RoPE append: layout may only set TMC_LAYOUT_X_PACKED.");
  int unroll, ks;
  default_packed(batch, n, 1, unroll, ks);
  if (norm) ks = n >= 16384 ? std::min(ks, kPackedNormWaves) : kPackedNormWaves;
  if (config && config->algorithm != 0) {
    unroll = config->unroll;
    ks = config->k_split;
  }
  TMC_REQUIRE((unroll == 1 || unroll == 2 || unroll == 4) && ks >= 1 &&
                  ks <= (norm ? kPackedNormWaves : 16),
              "Packed q.k.v RoPE append: config needs unroll 1|2|4 and k_split 1..16 (1..4 with "
              "RMSNorm).");
  RopeArgs ra;
  ra.cosine = cosine;
  ra.sine = sine;
  ra.valid_lengths = valid_lengths;
  ra.block_tables = block_tables;
  ra.active_count = active_count;
  ra.q_out = static_cast<half_t*>(q_out);
  ra.k_pool = static_cast<half_t*>(key_pool);
  ra.v_pool = static_cast<half_t*>(value_pool);
  ra.q_heads = (int)q_heads;
  ra.kv_heads = (int)kv_heads;
  ra.head_dim = (int)head_dim;
  ra.capacity = (int)capacity;
  ra.page_size = (int)page_size;
  ra.table_stride = (int)max_pages;
  const half_t* xs = static_cast<const half_t*>(x);
  const half_t* w = static_cast<const half_t*>(packed_w);
  half_t* none = static_cast<half_t*>(q_out);  // not written by the RoPE epilogue
  const hipStream_t st = as_stream(stream);
  PackedFuseArgs pf;
  pf.eps = eps;
  if (norm) {
    if (layout & TMC_LAYOUT_X_PACKED)
      return run_packed<1, half_t, true, false, true, kPackedNorm>(xs, w, w, none, batch, hidden,
                                                                   n, unroll, ks, st, ra, pf);
    return run_packed<1, half_t, false, false, true, kPackedNorm>(xs, w, w, none, batch, hidden, n,
                                                                  unroll, ks, st, ra, pf);
  }
  if (layout & TMC_LAYOUT_X_PACKED)
    return run_packed<1, half_t, true, false, true>(xs, w, w, none, batch, hidden, n, unroll, ks,
                                                    st, ra);
  return run_packed<1, half_t, false, false, true>(xs, w, w, none, batch, hidden, n, unroll, ks, st,
                                                   ra);
}

}  // namespace
}  // namespace tmc

extern "C" int tmc_qkv_rope_append_packed_f16(
    const void* x, const void* packed_w, const float* cosine, const float* sine,
    const int32_t* valid_lengths, const int32_t* block_tables, const int32_t* active_count,
    void* q_out, void* key_pool, void* value_pool, int64_t batch, int64_t hidden,
    int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t capacity, int64_t page_size,
    int64_t max_pages, int layout, const tmc_gemv_config* config, void* stream) {
  return qkv_rope_packed_entry(x, false, 0.0f, packed_w, cosine, sine, valid_lengths,
                               block_tables, active_count, q_out, key_pool, value_pool, batch,
                               hidden, q_heads, kv_heads, head_dim, capacity, page_size, max_pages,
                               layout, config, stream);
}

extern "C" int tmc_rmsnorm_qkv_rope_append_packed_f16(
    const void* x, const void* packed_w, const float* cosine, const float* sine,
    const int32_t* valid_lengths, const int32_t* block_tables, const int32_t* active_count,
    void* q_out, void* key_pool, void* value_pool, int64_t batch, int64_t hidden,
    int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t capacity, int64_t page_size,
    int64_t max_pages, float epsilon, int layout, const tmc_gemv_config* config, void* stream) {
  return qkv_rope_packed_entry(x, true, epsilon, packed_w, cosine, sine, valid_lengths,
                               block_tables, active_count, q_out, key_pool, value_pool, batch,
                               hidden, q_heads, kv_heads, head_dim, capacity, page_size, max_pages,
                               layout, config, stream);
}

extern "C" int tmc_gemm_packed_norm_f16(const void* x, const void* packed_w, void* y,
                                        int y_dtype, int64_t batch, int64_t in_features,
                                        int64_t out_features, float epsilon, int layout,
                                        const tmc_gemv_config* config, void* stream) {
  PackedFuseArgs pf;
  pf.eps = epsilon;
  return packed_entry(1, x, packed_w, nullptr, y, y_dtype, batch, in_features, out_features,
                      layout, config, stream, kPackedNorm, pf);
}

extern "C" int tmc_lm_head_partial_argmax_packed_norm_f16(
    const void* x, const void* packed_w, void* workspace, size_t workspace_bytes, int64_t batch,
    int64_t in_features, int64_t vocabulary, float epsilon, int layout,
    const tmc_gemv_config* config, void* stream) {
  const std::string what = "Packed LM head partial argmax";
  TMC_REQUIRE(x && packed_w && workspace, what + ": null device pointer.");
  TMC_REQUIRE(epsilon > 0.0f && std::isfinite(epsilon), what + ": epsilon must be positive.");
  TMC_REQUIRE(batch > 0 && in_features > 0 && vocabulary > 0 && batch < (1LL << 20) &&
                  vocabulary < (1LL << 28) && in_features % 8 == 0,
              what + ": dimensions must be positive and in_features a multiple of 8.");
  TMC_REQUIRE((layout & ~TMC_LAYOUT_X_PACKED) == 0,
              what + ": layout may only mark the input packed (TMC_LAYOUT_X_PACKED).");
  TMC_REQUIRE(workspace_bytes >= tmc_lm_head_argmax_workspace_bytes(batch, vocabulary),
              what + ": workspace is smaller than tmc_lm_head_argmax_workspace_bytes().");
  TMC_REQUIRE(aligned16(x) && aligned16(packed_w) && aligned16(workspace),
              what + ": operands must be 16-byte aligned.");
  TMC_REQUIRE((uint64_t)packed_elements(vocabulary, in_features) * 2 < kNone &&
                  (uint64_t)16 * in_features * 2 < kNone,
              what + ": operands exceed the 4 GiB buffer range.");
  int unroll, ks;
  default_packed(batch, vocabulary, 1, unroll, ks);
  ks = vocabulary >= 16384 ? std::min(ks, kPackedNormWaves) : kPackedNormWaves;
  if (vocabulary >= 16384) unroll = lm_head_unroll(batch);
  if (config && config->algorithm != 0) {
    unroll = config->unroll;
    ks = config->k_split;
  }
  TMC_REQUIRE((unroll == 1 || unroll == 2 || unroll == 4) && ks >= 1 && ks <= kPackedNormWaves,
              what + ": config needs unroll 1|2|4 and k_split 1..4.");
  PackedFuseArgs pf;
  pf.eps = epsilon;
  pf.argmax_rows = (int)batch;
  const half_t* xs = static_cast<const half_t*>(x);
  const half_t* w = static_cast<const half_t*>(packed_w);
  float* out = static_cast<float*>(workspace);
  const RopeArgs none{};
  if (layout & TMC_LAYOUT_X_PACKED)
    return run_packed<1, float, true, false, false, kPackedNorm, true>(
        xs, w, w, out, batch, in_features, vocabulary, unroll, ks, as_stream(stream), none, pf);
  return run_packed<1, float, false, false, false, kPackedNorm, true>(
      xs, w, w, out, batch, in_features, vocabulary, unroll, ks, as_stream(stream), none, pf);
}

extern "C" int tmc_gate_up_silu_packed_norm_f16(const void* x, const void* packed_gate,
                                                const void* packed_up, void* out, int64_t batch,
                                                int64_t hidden, int64_t intermediate,
                                                float epsilon, int layout,
                                                const tmc_gemv_config* config, void* stream) {
  PackedFuseArgs pf;
  pf.eps = epsilon;
  return packed_entry(2, x, packed_gate, packed_up, out, TMC_F16, batch, hidden, intermediate,
                      layout, config, stream, kPackedNorm, pf);
}

extern "C" int tmc_gemm_packed_residual_f16(const void* x, const void* packed_w,
                                            const void* residual, void* y, int64_t batch,
                                            int64_t in_features, int64_t out_features, int layout,
                                            const tmc_gemv_config* config, void* stream) {
  PackedFuseArgs pf;
  pf.residual = static_cast<const half_t*>(residual);
  return packed_entry(1, x, packed_w, nullptr, y, TMC_F16, batch, in_features, out_features,
                      layout, config, stream, kPackedResidual, pf);
}

extern "C" int tmc_gate_up_silu_packed_ex_f16(const void* x, const void* packed_gate,
                                              const void* packed_up, void* out, int64_t batch,
                                              int64_t hidden, int64_t intermediate, int layout,
                                              const tmc_gemv_config* config, void* stream) {
  return packed_entry(2, x, packed_gate, packed_up, out, TMC_F16, batch, hidden, intermediate,
                      layout, config, stream);
}

extern "C" int64_t tmc_packed_activation_elements(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return ((rows + 15) / 16) * ((cols + 31) / 32) * 512;
}

extern "C" int tmc_pack_activations_f16(const void* src, void* dst, int64_t rows, int64_t cols,
                                        int unpack, void* stream) {
  TMC_REQUIRE(src && dst, "Pack activations: null device pointer.");
  TMC_REQUIRE(rows > 0 && cols > 0 && cols % 8 == 0 && rows < (1LL << 31) && cols < (1LL << 31),
              "Pack activations: cols must be a positive multiple of 8.");
  TMC_REQUIRE(aligned16(src) && aligned16(dst), "Pack activations: operands must be 16-byte aligned.");
  const long slots = (long)(tmc_packed_activation_elements(rows, cols) / 8);
  const unsigned blocks = (unsigned)std::min<long>((slots + 255) / 256, 65536);
  hipLaunchKernelGGL(pack_activations_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                     static_cast<const half_t*>(src), static_cast<half_t*>(dst), (int)rows,
                     (int)cols, unpack, slots);
  return check_launch("pack_activations_kernel");
}
