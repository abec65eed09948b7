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

}  // namespace tmc
