// Device-side helpers shared by the gfx950 decode kernels.
//
// Wave64 conventions used throughout:
//  * a "row" is one DPP row of 16 lanes; row reductions use DPP
//    (quad_perm / row_half_mirror / row_mirror), which needs no LDS;
//  * reductions across rows use ds_bpermute (__shfl_xor) or v_readlane;
//  * every reduction is called with all 64 lanes active.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tmc {

typedef _Float16 half_t;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ------------------------------------------------------------------ loads
__device__ __forceinline__ h8 load_h8(const half_t* p) {
  return *reinterpret_cast<const h8*>(p);
}
// Streaming (read-once) 16-byte load: sets the non-temporal hint so weight
// streams do not evict reusable activations from the caches.
__device__ __forceinline__ h8 load_h8_stream(const half_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const h8*>(p));
}

// ------------------------------------------------------------------ conversions
template <typename T> __device__ __forceinline__ float to_float(T v);
template <> __device__ __forceinline__ float to_float<half_t>(half_t v) { return (float)v; }
template <> __device__ __forceinline__ float to_float<float>(float v) { return v; }

template <typename T> __device__ __forceinline__ T from_float(float v);
template <> __device__ __forceinline__ half_t from_float<half_t>(float v) { return (half_t)v; }
template <> __device__ __forceinline__ float from_float<float>(float v) { return v; }

// Round a float through the storage type (the reference kernels' `type(x)`).
template <typename T> __device__ __forceinline__ float through(float v) {
  return to_float<T>(from_float<T>(v));
}

// ------------------------------------------------------------------ dot products
// sum_{t<8} a[t]*b[t] + c with fp32 accumulation (v_dot2_f32_f16).
__device__ __forceinline__ float dot8(h8 a, h8 b, float c) {
  c = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 0, 1),
                             __builtin_shufflevector(b, b, 0, 1), c, false);
  c = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 2, 3),
                             __builtin_shufflevector(b, b, 2, 3), c, false);
  c = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 4, 5),
                             __builtin_shufflevector(b, b, 4, 5), c, false);
  c = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 6, 7),
                             __builtin_shufflevector(b, b, 6, 7), c, false);
  return c;
}

// ------------------------------------------------------------------ DPP
enum : int {
  kDppQuadSwap1 = 0xB1,     // quad_perm [1,0,3,2]
  kDppQuadSwap2 = 0x4E,     // quad_perm [2,3,0,1]
  kDppRowHalfMirror = 0x141,
  kDppRowMirror = 0x140,
};

template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N in {1,2,4,8,16}); every lane of a
// group receives the group total.
template <int N> __device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<kDppQuadSwap1>(v);
  if constexpr (N >= 4) v += dpp<kDppQuadSwap2>(v);
  if constexpr (N >= 8) v += dpp<kDppRowHalfMirror>(v);
  if constexpr (N >= 16) v += dpp<kDppRowMirror>(v);
  return v;
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Full wave sum, returned as a wave-uniform value.
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

// Combine lanes that differ in lane-index bits >= FROM (xor butterfly).
template <int FROM> __device__ __forceinline__ float cross_sum(float v) {
#pragma unroll
  for (int off = FROM; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
template <int FROM> __device__ __forceinline__ float cross_max(float v) {
#pragma unroll
  for (int off = FROM; off < kWave; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Greedy-token order (emitTokenArgmax, TransformerDecodeMetalEmitter.cpp:
// 198-256; emitLMHeadFinalArgmax, DecoderLLMMetalEmitter.cpp:730-753):
// candidate (cv, ci) replaces the best (bv, bi) when larger, or equal with a
// lower index; NaN never wins, and (-inf, -1) is the empty best.  The order
// is total on the candidates it accepts, so any reduction tree over the
// vocabulary gives the sequential scan's token.
__device__ __forceinline__ bool argmax_better(float cv, int ci, float bv, int bi) {
  return cv > bv || (cv == bv && ci >= 0 && (bi < 0 || ci < bi));
}

// Wave-wide argmax of (best, selected): every lane receives the winner.
__device__ __forceinline__ void argmax_wave(float& best, int& selected) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(selected, off, kWave);
    if (argmax_better(ov, oi, best, selected)) {
      best = ov;
      selected = oi;
    }
  }
}

// Partial-argmax workspace of the token-only LM heads: int32 count of
// partials per row at the start, fp32 values [rows][cap] from byte 256, then
// int32 indices [rows][cap].
struct ArgmaxPartials {
  int* count;
  float* values;
  int* indices;
  int cap;
};
__device__ __forceinline__ ArgmaxPartials argmax_partials(void* workspace, int rows, int cap) {
  char* base = static_cast<char*>(workspace);
  ArgmaxPartials a;
  a.count = reinterpret_cast<int*>(base);
  a.values = reinterpret_cast<float*>(base + 256);
  a.indices = reinterpret_cast<int*>(base + 256 + (size_t)rows * cap * sizeof(float));
  a.cap = cap;
  return a;
}

// Workgroup barrier ordering LDS only (__syncthreads() also waits for every
// outstanding global load, e.g. for a weight stream still in flight).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Raw buffer loads: an offset at or past the resource's byte count reads as
// zero, so an absent element needs a select, not a branch.
constexpr unsigned kBufferAbsent = 0xFFFFFFF0u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_resource(const void* base,
                                                                  unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ h8 buffer_load_h8(__amdgpu_buffer_rsrc_t r, unsigned byte_offset) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, 0));
}

// Interleaved pair rotation shared by every RoPE kernel and the fused q.k.v
// projection epilogue, written with explicit fused multiply-adds so that all
// of them produce the same bits for the same pair.
__device__ __forceinline__ void rotate_pair(float even, float odd, float c, float s,
                                            float& out_even, float& out_odd) {
  out_even = __fmaf_rn(even, c, -(odd * s));
  out_odd = __fmaf_rn(even, s, odd * c);
}

// Epilogue of a q.k.v projection fused with RoPE and the paged K/V append:
// output features 2i, 2i+1 of a request's projection row are one
// interleaved RoPE pair of q or k, or two v features.  The pair is rounded
// to fp16 as the projection output would be, rotated as
// decode_rope_append_kernel rotates it, and stored where that kernel stores
// it: q to q_out[request], k and v into the pools at position
// valid_lengths[request] - 1 through block_tables + request * table_stride.
// Requests at or past active_count[0], lengths outside [1, capacity] and
// missing pages are skipped.
struct RopeArgs {
  const float* cosine = nullptr;
  const float* sine = nullptr;
  const int32_t* valid_lengths = nullptr;
  const int32_t* block_tables = nullptr;
  const int32_t* active_count = nullptr;
  half_t* q_out = nullptr;
  half_t* k_pool = nullptr;
  half_t* v_pool = nullptr;
  int q_heads = 0, kv_heads = 0, head_dim = 0, capacity = 0, page_size = 0, table_stride = 0;
  int request_base = 0;  // request index of a kernel's first batch row
};

__device__ __forceinline__ void rope_append_pair(const RopeArgs& ra, int request, int column,
                                                 float sum_even, float sum_odd) {
  const int valid = ra.valid_lengths[request];
  if (request >= ra.active_count[0] || valid <= 0 || valid > ra.capacity) return;
  const int position = valid - 1;
  const int d = ra.head_dim, pairs = d / 2;
  const int q_width = ra.q_heads * d, kv_width = ra.kv_heads * d;
  const half_t x0 = from_float<half_t>(sum_even), x1 = from_float<half_t>(sum_odd);
  half_t y0 = x0, y1 = x1;
  if (column < q_width + kv_width) {
    const int pair = (column % d) / 2;
    const float c = ra.cosine[(size_t)position * pairs + pair];
    const float s = ra.sine[(size_t)position * pairs + pair];
    float re, ro;
    rotate_pair(to_float<half_t>(x0), to_float<half_t>(x1), c, s, re, ro);
    // the fp32 results are rounded once to fp16, as the unfused kernel does
    asm volatile("" : "+v"(re), "+v"(ro));
    y0 = from_float<half_t>(re);
    y1 = from_float<half_t>(ro);
  }
  half_t* dst;
  if (column < q_width) {
    dst = ra.q_out + (size_t)request * q_width + column;
  } else {
    const int page =
        ra.block_tables[(size_t)request * ra.table_stride + position / ra.page_size];
    if (page < 0) return;
    const bool key = column < q_width + kv_width;
    const int feature = column - q_width - (key ? 0 : kv_width);
    dst = (key ? ra.k_pool : ra.v_pool) +
          (((size_t)page * ra.kv_heads + feature / d) * ra.page_size + position % ra.page_size) * d +
          feature % d;
  }
  dst[0] = y0;
  dst[1] = y1;
}

}  // namespace tmc
