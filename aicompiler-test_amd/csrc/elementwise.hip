// Row reductions and elementwise decode kernels for gfx950:
// RMSNorm, Add+RMSNorm, SiLU*Mul, residual add, embedding gather, RoPE,
// KV-cache appends (contiguous, paged, serving), argmax, synthetic fill and
// a copy probe.  Each kernel keeps the reference kernel's arithmetic and
// rounding points (cited per kernel); launch shapes are chosen for wave64.
#include "tmc_abi.hpp"
#include "tmc_device.hpp"

namespace tmc {
namespace {

constexpr int kThreads = 256;

// Block-wide sum for THREADS threads (a multiple of 64); every thread gets
// the total.
template <int THREADS = kThreads>
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  constexpr int waves = THREADS / kWave;
  v = wave_sum(v);
  if ((threadIdx.x & (kWave - 1)) == 0) scratch[threadIdx.x / kWave] = v;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < waves; ++i) total += scratch[i];
  return total;
}

// emitDecoderRMSNorm (DecoderLLMMetalEmitter.cpp:63-108): fp32 sum of
// squares, inverse = rsqrt(sum/width + eps), y = T(x * inverse * w).  Two
// passes over the row; at 256 threads this is the tuner's fixed baseline
// (emitRMSNormBaseline, RMSNormBaseline.cpp:13-72).
template <typename T, int THREADS = kThreads>
__global__ __launch_bounds__(THREADS) void rmsnorm_kernel(const T* __restrict__ x,
                                                         const T* __restrict__ w,
                                                         T* __restrict__ y, int width,
                                                         float eps) {
  __shared__ float scratch[THREADS / kWave];
  const size_t base = (size_t)blockIdx.x * width;
  float squares = 0.0f;
  for (int i = threadIdx.x; i < width; i += THREADS) {
    const float v = to_float<T>(x[base + i]);
    squares += v * v;
  }
  const float total = block_sum<THREADS>(squares, scratch);
  const float inverse = 1.0f / sqrtf(total / (float)width + eps);
  for (int i = threadIdx.x; i < width; i += THREADS)
    y[base + i] = from_float<T>(to_float<T>(x[base + i]) * inverse * to_float<T>(w[i]));
}

// emitDecoderResidualRMSNorm (DecoderLLMMetalEmitter.cpp:417-477).
template <typename T, int THREADS = kThreads>
__global__ __launch_bounds__(THREADS) void add_rmsnorm_kernel(
    const T* __restrict__ residual, const T* __restrict__ update, const T* __restrict__ w,
    T* __restrict__ sum_out, T* __restrict__ norm_out, int width, float eps) {
  __shared__ float scratch[THREADS / kWave];
  const size_t base = (size_t)blockIdx.x * width;
  float squares = 0.0f;
  for (int i = threadIdx.x; i < width; i += THREADS) {
    const float v = through<T>(to_float<T>(residual[base + i]) + to_float<T>(update[base + i]));
    sum_out[base + i] = from_float<T>(v);
    squares += v * v;
  }
  const float total = block_sum<THREADS>(squares, scratch);
  const float inverse = 1.0f / sqrtf(total / (float)width + eps);
  for (int i = threadIdx.x; i < width; i += THREADS) {
    const float v = through<T>(to_float<T>(residual[base + i]) + to_float<T>(update[base + i]));
    norm_out[base + i] = from_float<T>(v * inverse * to_float<T>(w[i]));
  }
}

// Register-resident variants for rows of at most kMaxVec * 8 * THREADS
// elements with vector-aligned rows: each thread loads its 8-element
// slices once, the row is reduced once, and the outputs are written from
// registers (one global read pass instead of two).
constexpr int kMaxVec = 4;

template <typename T> struct Vec8;
template <> struct Vec8<half_t> { typedef h8 type; };
template <> struct Vec8<float> { typedef float type __attribute__((ext_vector_type(8))); };

// POUT: the normalized row is written in the activation fragment order of
// the packed GEMM (include/tmc_hip.h): 16-row pass r / 16, 32-k chunk
// v / 4, lane r % 16 + 16 * (v % 4) for the 8 elements 8v..8v+7.
template <typename T, int NV, bool ADD, int THREADS, bool POUT = false>
__global__ __launch_bounds__(THREADS) void norm_vec_kernel(const T* __restrict__ residual,
                                                          const T* __restrict__ update,
                                                          const T* __restrict__ w,
                                                          T* __restrict__ sum_out,
                                                          T* __restrict__ norm_out, int width,
                                                          float eps) {
  typedef typename Vec8<T>::type V;
  __shared__ float scratch[THREADS / kWave];
  const size_t base = (size_t)blockIdx.x * width;
  const int vecs = width / 8;
  V val[NV], wv[NV];
  float squares = 0.0f;
  // gamma is loaded with the row, so the reduction is the only wait
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = threadIdx.x + i * THREADS;
    if (v < vecs) wv[i] = *reinterpret_cast<const V*>(w + 8 * v);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = threadIdx.x + i * THREADS;
    if (v < vecs) {
      V a = *reinterpret_cast<const V*>(residual + base + 8 * v);
      if constexpr (ADD) {
        const V b = *reinterpret_cast<const V*>(update + base + 8 * v);
#pragma unroll
        for (int t = 0; t < 8; ++t) a[t] = from_float<T>(to_float<T>(a[t]) + to_float<T>(b[t]));
      }
      val[i] = a;
#pragma unroll
      for (int t = 0; t < 8; ++t) squares += to_float<T>(a[t]) * to_float<T>(a[t]);
    }
  }
  const float total = block_sum<THREADS>(squares, scratch);
  const float inverse = 1.0f / sqrtf(total / (float)width + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = threadIdx.x + i * THREADS;
    if (v < vecs) {
      V n;
#pragma unroll
      for (int t = 0; t < 8; ++t)
        n[t] = from_float<T>(to_float<T>(val[i][t]) * inverse * to_float<T>(wv[i][t]));
      if constexpr (ADD) *reinterpret_cast<V*>(sum_out + base + 8 * v) = val[i];
      if constexpr (POUT) {
        const size_t chunks = (size_t)(width + 31) / 32;
        const size_t slot = ((size_t)(blockIdx.x >> 4) * chunks + (size_t)(v >> 2)) * 64 +
                            (blockIdx.x & 15) + 16 * (v & 3);
        *reinterpret_cast<V*>(norm_out + slot * 8) = n;
      } else {
        *reinterpret_cast<V*>(norm_out + base + 8 * v) = n;
      }
    }
  }
}

// RMSNorm / Add+RMSNorm (fp16, 256 threads) with the normalized row written
// in the packed activation order; false when the row does not fit the
// register-resident kernel.
template <bool ADD>
bool launch_norm_packed_out(const half_t* r, const half_t* u, const half_t* w, half_t* s,
                            half_t* n, int64_t rows, int64_t width, float eps,
                            hipStream_t stream) {
  if (width % 8 != 0) return false;
  const dim3 grid((unsigned)rows);
  if (width / 8 == 512) {
    // width 4096: one 16-byte chunk per thread at 512 threads (the rows are
    // latency bound; ~0.5 us shorter than 2 chunks x 256 threads)
    hipLaunchKernelGGL((norm_vec_kernel<half_t, 1, ADD, 512, true>), grid, dim3(512), 0, stream,
                       r, u, w, s, n, (int)width, eps);
    return true;
  }
  const int nv = (int)((width / 8 + kThreads - 1) / kThreads);
  const dim3 block(kThreads);
  switch (nv) {
  case 1: hipLaunchKernelGGL((norm_vec_kernel<half_t, 1, ADD, kThreads, true>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); return true;
  case 2: hipLaunchKernelGGL((norm_vec_kernel<half_t, 2, ADD, kThreads, true>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); return true;
  case 3: hipLaunchKernelGGL((norm_vec_kernel<half_t, 3, ADD, kThreads, true>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); return true;
  case 4: hipLaunchKernelGGL((norm_vec_kernel<half_t, 4, ADD, kThreads, true>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); return true;
  default: return false;
  }
}

template <typename T, bool ADD, int THREADS>
bool launch_norm_vec(const T* r, const T* u, const T* w, T* s, T* n, int64_t rows, int64_t width,
                     float eps, hipStream_t stream) {
  constexpr uintptr_t align = sizeof(typename Vec8<T>::type);
  auto ok = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % align) == 0; };
  if (width % 8 != 0 || !ok(r) || !ok(w) || !ok(n) || (ADD && (!ok(u) || !ok(s)))) return false;
  const int64_t vecs = width / 8;
  const int nv = (int)((vecs + THREADS - 1) / THREADS);
  if (nv > kMaxVec) return false;
  const dim3 grid((unsigned)rows), block(THREADS);
  switch (nv) {
  case 1: hipLaunchKernelGGL((norm_vec_kernel<T, 1, ADD, THREADS>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); break;
  case 2: hipLaunchKernelGGL((norm_vec_kernel<T, 2, ADD, THREADS>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); break;
  case 3: hipLaunchKernelGGL((norm_vec_kernel<T, 3, ADD, THREADS>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); break;
  default: hipLaunchKernelGGL((norm_vec_kernel<T, 4, ADD, THREADS>), grid, block, 0, stream, r, u, w, s, n, (int)width, eps); break;
  }
  return true;
}

// One RMSNorm / Add+RMSNorm launch at THREADS threads per row: the
// register-resident kernel when the row fits (unless two_pass), else the
// two-pass kernel.
template <typename T, bool ADD, int THREADS>
void launch_norm(const T* r, const T* u, const T* w, T* s, T* n, int64_t rows, int64_t width,
                 float eps, bool two_pass, hipStream_t stream) {
  if (!two_pass && launch_norm_vec<T, ADD, THREADS>(r, u, w, s, n, rows, width, eps, stream))
    return;
  if constexpr (ADD)
    hipLaunchKernelGGL((add_rmsnorm_kernel<T, THREADS>), dim3((unsigned)rows), dim3(THREADS), 0,
                       stream, r, u, w, s, n, (int)width, eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<T, THREADS>), dim3((unsigned)rows), dim3(THREADS), 0,
                       stream, r, w, n, (int)width, eps);
}

template <typename T, bool ADD>
bool launch_norm_threads(const T* r, const T* u, const T* w, T* s, T* n, int64_t rows,
                         int64_t width, float eps, int threads, bool two_pass,
                         hipStream_t stream) {
  switch (threads) {
  case 64: launch_norm<T, ADD, 64>(r, u, w, s, n, rows, width, eps, two_pass, stream); return true;
  case 128: launch_norm<T, ADD, 128>(r, u, w, s, n, rows, width, eps, two_pass, stream); return true;
  case 256: launch_norm<T, ADD, 256>(r, u, w, s, n, rows, width, eps, two_pass, stream); return true;
  case 512: launch_norm<T, ADD, 512>(r, u, w, s, n, rows, width, eps, two_pass, stream); return true;
  case 1024: launch_norm<T, ADD, 1024>(r, u, w, s, n, rows, width, eps, two_pass, stream); return true;
  default: return false;
  }
}

// emitDecoderSiLUMul (DecoderLLMMetalEmitter.cpp:395-415).
template <typename T>
__device__ __forceinline__ T silu_mul_one(T gate, T up) {
  const float g = to_float<T>(gate);
  const float activated = through<T>(g / (1.0f + expf(-g)));
  return from_float<T>(activated * to_float<T>(up));
}

template <typename T>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const T* __restrict__ gate,
                                                           const T* __restrict__ up,
                                                           T* __restrict__ out, size_t count) {
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (size_t)gridDim.x * kThreads)
    out[i] = silu_mul_one<T>(gate[i], up[i]);
}

// fp16, 16-byte aligned, count % 8 == 0: eight elements per thread with
// 16-byte loads and stores (same per-element arithmetic).
__global__ __launch_bounds__(kThreads) void silu_mul_h8_kernel(const h8* __restrict__ gate,
                                                              const h8* __restrict__ up,
                                                              h8* __restrict__ out, size_t vectors) {
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < vectors;
       i += (size_t)gridDim.x * kThreads) {
    const h8 g = gate[i], u = up[i];
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = silu_mul_one<half_t>(g[e], u[e]);
    out[i] = r;
  }
}

// emitDecoderAdd (DecoderLLMMetalEmitter.cpp:375-393).
template <typename T>
__global__ __launch_bounds__(kThreads) void add_kernel(const T* __restrict__ a,
                                                      const T* __restrict__ b,
                                                      T* __restrict__ out, size_t count) {
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (size_t)gridDim.x * kThreads)
    out[i] = from_float<T>(to_float<T>(a[i]) + to_float<T>(b[i]));
}

// Element-wise operations of the graph path (TensorIR Add, Mul, SiLU and the
// fused SiLU + Mul region, FusionMetalEmitter.cpp:103-210 in the reference),
// for any workgroup size: one element per thread per grid stride.  SiLU
// rounds its activation to T before a multiply, as a stored SiLU output
// would be, so the fused form equals SiLU followed by Mul bit for bit.
enum EwOp { kEwAdd = 0, kEwMul = 1, kEwSilu = 2, kEwSiluMul = 3 };

template <typename T, int OP>
__global__ __launch_bounds__(kThreads) void elementwise_kernel(const T* __restrict__ a,
                                                              const T* __restrict__ b,
                                                              T* __restrict__ out, size_t count) {
  const size_t step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += step) {
    const float x = to_float<T>(a[i]);
    if constexpr (OP == kEwAdd) out[i] = from_float<T>(x + to_float<T>(b[i]));
    if constexpr (OP == kEwMul) out[i] = from_float<T>(x * to_float<T>(b[i]));
    if constexpr (OP == kEwSilu) out[i] = from_float<T>(x / (1.0f + expf(-x)));
    if constexpr (OP == kEwSiluMul) out[i] = silu_mul_one<T>(a[i], b[i]);
  }
}

// emitDecoderEmbedding (DecoderLLMMetalEmitter.cpp:35-61).
template <typename T>
__global__ __launch_bounds__(kThreads) void embedding_kernel(const int32_t* __restrict__ tokens,
                                                            const T* __restrict__ table,
                                                            T* __restrict__ out, int hidden,
                                                            int vocabulary) {
  const int row = blockIdx.y;
  const int token = tokens[row];
  if (token < 0 || token >= vocabulary) return;
  for (int f = blockIdx.x * kThreads + threadIdx.x; f < hidden; f += gridDim.x * kThreads)
    out[(size_t)row * hidden + f] = table[(size_t)token * hidden + f];
}

// emitDecoderRoPE (DecoderLLMMetalEmitter.cpp:110-158).
template <typename T>
__global__ __launch_bounds__(kThreads) void rope_kernel(const T* __restrict__ x,
                                                       const float* __restrict__ cosine,
                                                       const float* __restrict__ sine,
                                                       const int32_t* __restrict__ valid_length,
                                                       T* __restrict__ out, int batch, int seq,
                                                       int heads, int head_dim, int capacity) {
  const int pairs = head_dim / 2;
  const long items = (long)batch * heads * seq * pairs;
  const long gid = (long)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= items) return;
  const int valid = valid_length[0];
  if (valid < seq || valid > capacity) return;
  const int pair = (int)(gid % pairs);
  const int token = (int)((gid / pairs) % seq);
  const int head = (int)((gid / ((long)pairs * seq)) % heads);
  const int b = (int)(gid / ((long)pairs * seq * heads));
  const int position = valid - seq + token;
  const size_t hidden = (size_t)heads * head_dim;
  const size_t in_base = ((size_t)b * seq + token) * hidden + (size_t)head * head_dim + 2 * pair;
  const size_t out_base = (((size_t)b * heads + head) * seq + token) * head_dim + 2 * pair;
  const float c = cosine[(size_t)position * pairs + pair];
  const float s = sine[(size_t)position * pairs + pair];
  float re, ro;
  rotate_pair(to_float<T>(x[in_base]), to_float<T>(x[in_base + 1]), c, s, re, ro);
  out[out_base] = from_float<T>(re);
  out[out_base + 1] = from_float<T>(ro);
}

// emitServingRoPE (DecoderLLMMetalEmitter.cpp:260-312).
template <typename T>
__global__ __launch_bounds__(kThreads) void serving_rope_kernel(
    const T* __restrict__ x, const float* __restrict__ cosine, const float* __restrict__ sine,
    const int32_t* __restrict__ valid_lengths, const int32_t* __restrict__ active_count,
    T* __restrict__ out, int max_batch, int heads, int head_dim, int capacity) {
  const int pairs = head_dim / 2;
  const long per_request = (long)heads * pairs;
  const long gid = (long)blockIdx.x * kThreads + threadIdx.x;
  const long request = gid / per_request;
  if (gid >= (long)max_batch * per_request || request >= active_count[0]) return;
  const int pair = (int)(gid % pairs);
  const int head = (int)((gid / pairs) % heads);
  const int valid = valid_lengths[request];
  if (valid <= 0 || valid > capacity) return;
  const int position = valid - 1;
  const size_t base = ((size_t)request * heads + head) * head_dim + 2 * pair;
  const float c = cosine[(size_t)position * pairs + pair];
  const float s = sine[(size_t)position * pairs + pair];
  float re, ro;
  rotate_pair(to_float<T>(x[base]), to_float<T>(x[base + 1]), c, s, re, ro);
  out[base] = from_float<T>(re);
  out[base + 1] = from_float<T>(ro);
}

// emitDecoderCacheAppend / emitDecoderPagedCacheAppend
// (DecoderLLMMetalEmitter.cpp:160-258): bit copies, one element per thread.
template <typename T, bool PAGED>
__global__ __launch_bounds__(kThreads) void append_kernel(
    const T* __restrict__ input, const int32_t* __restrict__ valid_length,
    const int32_t* __restrict__ block_table, T* __restrict__ cache, int batch, int seq,
    int heads, int head_dim, int capacity, int page_size, int head_major) {
  const long hidden = (long)heads * head_dim;
  const long items = (long)batch * seq * hidden;
  const long gid = (long)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= items) return;
  const int valid = valid_length[0];
  if (valid < seq || valid > capacity) return;
  const long feature = gid % hidden;
  const int token = (int)((gid / hidden) % seq);
  const int b = (int)(gid / (hidden * seq));
  const int head = (int)(feature / head_dim);
  const int component = (int)(feature % head_dim);
  const int position = valid - seq + token;
  size_t dst;
  if constexpr (PAGED) {
    const int page = block_table[position / page_size];
    if (page < 0) return;
    dst = ((((size_t)page * batch + b) * heads + head) * page_size + position % page_size) *
              head_dim + component;
  } else {
    dst = (((size_t)b * heads + head) * capacity + position) * head_dim + component;
  }
  const size_t src = head_major ? (((size_t)b * heads + head) * seq + token) * head_dim + component
                                : ((size_t)b * seq + token) * hidden + feature;
  cache[dst] = input[src];
}

// emitServingPagedCacheAppend (DecoderLLMMetalEmitter.cpp:314-373).
template <typename T>
__global__ __launch_bounds__(kThreads) void serving_append_kernel(
    const T* __restrict__ input, const int32_t* __restrict__ valid_lengths,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ active_count,
    T* __restrict__ cache, int max_batch, int heads, int head_dim, int capacity, int page_size,
    int head_major) {
  const long hidden = (long)heads * head_dim;
  const long gid = (long)blockIdx.x * kThreads + threadIdx.x;
  const long request = gid / hidden;
  if (gid >= (long)max_batch * hidden || request >= active_count[0]) return;
  const long feature = gid % hidden;
  const int head = (int)(feature / head_dim);
  const int component = (int)(feature % head_dim);
  const int valid = valid_lengths[request];
  if (valid <= 0 || valid > capacity) return;
  const int position = valid - 1;
  const int max_pages = (capacity + page_size - 1) / page_size;
  const int page = block_tables[request * max_pages + position / page_size];
  if (page < 0) return;
  const size_t dst =
      (((size_t)page * heads + head) * page_size + position % page_size) * head_dim + component;
  const size_t src = head_major ? ((size_t)request * heads + head) * head_dim + component
                                : (size_t)request * hidden + feature;
  cache[dst] = input[src];
}

// Decode-step fusion of emitServingRoPE (DecoderLLMMetalEmitter.cpp:260-312)
// for the query and key heads with emitServingPagedCacheAppend (:314-373) for
// the rotated key and the value, reading one fused q|k|v projection row per
// request: row b = [q heads | kv key heads | kv value heads] x head_dim.  One
// thread moves one interleaved pair.  The rotated query goes to q_out
// [max_batch, q_heads * head_dim]; the rotated key and the value are stored
// at position valid_lengths[b] - 1 of the pools [page][kv_heads][page_size]
// [head_dim] through block_tables[b * table_stride + position / page_size]
// (table_stride = max_pages, or 0 when every row is a token of one request).
// Rows at or beyond active_count[0], rows whose length is outside
// [1, capacity] and positions whose page entry is negative are skipped.
template <typename T>
__global__ __launch_bounds__(kThreads) void decode_rope_append_kernel(
    const T* __restrict__ qkv, const float* __restrict__ cosine, const float* __restrict__ sine,
    const int32_t* __restrict__ valid_lengths, const int32_t* __restrict__ block_tables,
    const int32_t* __restrict__ active_count, T* __restrict__ q_out, T* __restrict__ k_pool,
    T* __restrict__ v_pool, int max_batch, int q_heads, int kv_heads, int head_dim, int capacity,
    int page_size, int table_stride, const int32_t* __restrict__ row_table, int table_rows) {
  const int pairs = head_dim / 2;
  const int row_pairs = (q_heads + 2 * kv_heads) * pairs;
  const long gid = (long)blockIdx.x * kThreads + threadIdx.x;
  const int request = (int)(gid / row_pairs);
  if (request >= max_batch) return;
  // The active count, the row's length and its q.k.v pair are read together
  // (all in bounds for request < max_batch), so the tables are the only
  // dependent round trip.
  const int active = active_count[0];
  const int valid = valid_lengths[request];
  const int column = 2 * (int)(gid % row_pairs);
  const int q_width = q_heads * head_dim, kv_width = kv_heads * head_dim;
  const T* src = qkv + (size_t)request * (q_width + 2 * kv_width) + column;
  const T x0 = src[0], x1 = src[1];
  if (request >= active || valid <= 0 || valid > capacity) return;
  const int position = valid - 1;
  // Table row: the row table's entry (several requests in one prefill
  // chunk), else the request itself (table_stride 0: one shared table).
  const int trow = row_table ? row_table[request] : request;
  if (row_table && (trow < 0 || trow >= table_rows)) return;
  const int pair = (column % head_dim) / 2;
  if (column < q_width + kv_width) {
    const float c = cosine[(size_t)position * pairs + pair];
    const float s = sine[(size_t)position * pairs + pair];
    float re, ro;
    rotate_pair(to_float<T>(x0), to_float<T>(x1), c, s, re, ro);
    if (column < q_width) {
      T* dst = q_out + (size_t)request * q_width + column;
      dst[0] = from_float<T>(re);
      dst[1] = from_float<T>(ro);
      return;
    }
    const int page = block_tables[(size_t)trow * table_stride + position / page_size];
    if (page < 0) return;
    const int feature = column - q_width;
    T* dst = k_pool + (((size_t)page * kv_heads + feature / head_dim) * page_size +
                       position % page_size) * head_dim + feature % head_dim;
    dst[0] = from_float<T>(re);
    dst[1] = from_float<T>(ro);
    return;
  }
  const int page = block_tables[(size_t)trow * table_stride + position / page_size];
  if (page < 0) return;
  const int feature = column - q_width - kv_width;
  T* dst = v_pool + (((size_t)page * kv_heads + feature / head_dim) * page_size +
                     position % page_size) * head_dim + feature % head_dim;
  dst[0] = x0;
  dst[1] = x1;
}

// fp16 with head_dim % 8 == 0 and 16-byte aligned buffers: one thread per
// 8 consecutive elements (4 interleaved pairs of one head) with 16-byte
// loads and stores; the rotation is rotate_pair, so the bits match the
// one-pair kernel.
__global__ __launch_bounds__(kThreads) void decode_rope_append_h8_kernel(
    const half_t* __restrict__ qkv, const float* __restrict__ cosine,
    const float* __restrict__ sine, const int32_t* __restrict__ valid_lengths,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ active_count,
    half_t* __restrict__ q_out, half_t* __restrict__ k_pool, half_t* __restrict__ v_pool,
    int max_batch, int q_heads, int kv_heads, int head_dim, int capacity, int page_size,
    int table_stride, const int32_t* __restrict__ row_table, int table_rows) {
  const int pairs = head_dim / 2;
  const int row_octs = (q_heads + 2 * kv_heads) * head_dim / 8;
  const long gid = (long)blockIdx.x * kThreads + threadIdx.x;
  const int request = (int)(gid / row_octs);
  if (request >= max_batch) return;
  const int active = active_count[0];
  const int valid = valid_lengths[request];
  const int column = 8 * (int)(gid % row_octs);
  const int q_width = q_heads * head_dim, kv_width = kv_heads * head_dim;
  const h8 x = *reinterpret_cast<const h8*>(qkv + (size_t)request * (q_width + 2 * kv_width) + column);
  if (request >= active || valid <= 0 || valid > capacity) return;
  const int position = valid - 1;
  // Table row: the row table's entry (several requests in one prefill
  // chunk), else the request itself (table_stride 0: one shared table).
  const int trow = row_table ? row_table[request] : request;
  if (row_table && (trow < 0 || trow >= table_rows)) return;
  if (column < q_width + kv_width) {
    const int pair0 = (column % head_dim) / 2;
    const f4 c = *reinterpret_cast<const f4*>(cosine + (size_t)position * pairs + pair0);
    const f4 sn = *reinterpret_cast<const f4*>(sine + (size_t)position * pairs + pair0);
    h8 y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float re, ro;
      rotate_pair((float)x[2 * i], (float)x[2 * i + 1], c[i], sn[i], re, ro);
      // Round to fp32 first, then to fp16, as the one-pair kernels do: keep
      // the compiler from folding the fma and the conversion into one
      // mixed-precision op that rounds once.
      asm volatile("" : "+v"(re), "+v"(ro));
      y[2 * i] = (half_t)re;
      y[2 * i + 1] = (half_t)ro;
    }
    if (column < q_width) {
      *reinterpret_cast<h8*>(q_out + (size_t)request * q_width + column) = y;
      return;
    }
    const int page = block_tables[(size_t)trow * table_stride + position / page_size];
    if (page < 0) return;
    const int feature = column - q_width;
    *reinterpret_cast<h8*>(k_pool + (((size_t)page * kv_heads + feature / head_dim) * page_size +
                                     position % page_size) * head_dim + feature % head_dim) = y;
    return;
  }
  const int page = block_tables[(size_t)trow * table_stride + position / page_size];
  if (page < 0) return;
  const int feature = column - q_width - kv_width;
  *reinterpret_cast<h8*>(v_pool + (((size_t)page * kv_heads + feature / head_dim) * page_size +
                                   position % page_size) * head_dim + feature % head_dim) = x;
}

__device__ __forceinline__ bool better(float cv, int ci, float bv, int bi) {
  return argmax_better(cv, ci, bv, bi);
}

// emitTokenArgmax (TransformerDecodeMetalEmitter.cpp:198-256): greedy
// token, ties to the lowest index, NaN never selected.  One 1024-thread block
// per row; each thread issues all of its 16-byte loads (up to kArgmaxLoads)
// before comparing, so a 32000-entry row costs one memory round trip.
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxLoads = 8;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ logits,
                                                               int32_t* __restrict__ tokens,
                                                               int vocabulary) {
  __shared__ float best_v[kArgmaxThreads / kWave];
  __shared__ int best_i[kArgmaxThreads / kWave];
  const float* row = logits + (size_t)blockIdx.x * vocabulary;
  float best = -INFINITY;
  int selected = -1;
  const bool vec = (vocabulary & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0;
  if (vec) {
    const int quads = vocabulary >> 2;
    for (int q0 = threadIdx.x; q0 < quads; q0 += kArgmaxThreads * kArgmaxLoads) {
      float4 v[kArgmaxLoads];
#pragma unroll
      for (int u = 0; u < kArgmaxLoads; ++u) {
        const int q = q0 + u * kArgmaxThreads;
        v[u] = q < quads ? reinterpret_cast<const float4*>(row)[q]
                         : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      }
#pragma unroll
      for (int u = 0; u < kArgmaxLoads; ++u) {
        const int t = 4 * (q0 + u * kArgmaxThreads);
        const float c[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t + e < vocabulary && (c[e] > best || (c[e] == best && (selected < 0 || t + e < selected)))) {
            best = c[e];
            selected = t + e;
          }
      }
    }
  } else {
    for (int t = threadIdx.x; t < vocabulary; t += kArgmaxThreads) {
      const float c = row[t];
      if (c > best || (c == best && (selected < 0 || t < selected))) {
        best = c;
        selected = t;
      }
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(selected, off, kWave);
    if (better(ov, oi, best, selected)) {
      best = ov;
      selected = oi;
    }
  }
  if ((threadIdx.x & (kWave - 1)) == 0) {
    best_v[threadIdx.x / kWave] = best;
    best_i[threadIdx.x / kWave] = selected;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = best_v[0];
    int bi = best_i[0];
    for (int w = 1; w < kArgmaxThreads / kWave; ++w)
      if (better(best_v[w], best_i[w], bv, bi)) {
        bv = best_v[w];
        bi = best_i[w];
      }
    tokens[blockIdx.x] = bi;
  }
}

// Counter-based N(mean, std) generator: splitmix64 of (seed, index) gives two
// uniforms per pair of outputs, Box-Muller maps them to normals.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void fill_normal_kernel(T* __restrict__ out, size_t count,
                                                              uint64_t seed, float mean,
                                                              float std) {
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (size_t)gridDim.x * kThreads) {
    const uint64_t pair = i >> 1;
    const uint64_t a = splitmix64(seed * 0xD1B54A32D192ED03ull + 2 * pair);
    const uint64_t b = splitmix64(seed * 0xD1B54A32D192ED03ull + 2 * pair + 1);
    const float u1 = ((float)(a >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)(b >> 40) * (1.0f / 16777216.0f);           // [0, 1)
    const float r = sqrtf(-2.0f * logf(u1));
    const float angle = 6.283185307179586f * u2;
    const float z = (i & 1) ? r * sinf(angle) : r * cosf(angle);
    out[i] = from_float<T>(mean + std * z);
  }
}

__global__ __launch_bounds__(kThreads) void copy_kernel(const uint4* __restrict__ src,
                                                       uint4* __restrict__ dst, size_t count) {
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (size_t)gridDim.x * kThreads)
    dst[i] = src[i];
}

// Read-only stream: 4096 blocks, each a contiguous share of the buffer, four
// 16-byte non-temporal loads per lane in flight; the sink is written only
// when a block's sum hits a fixed constant, so the loads cannot be dropped.
constexpr int kReadProbeBlocks = 4096;
constexpr int kReadProbeDepth = 4;
typedef float probe_f4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void read_probe_kernel(const probe_f4* __restrict__ src,
                                                         float* __restrict__ sink, size_t count,
                                                         size_t per_block) {
  const size_t base = (size_t)blockIdx.x * per_block;
  float acc = 0.0f;
  for (size_t i = threadIdx.x; i < per_block; i += 256 * kReadProbeDepth) {
    probe_f4 v[kReadProbeDepth];
#pragma unroll
    for (int d = 0; d < kReadProbeDepth; ++d) {
      const size_t at = i + 256 * (size_t)d;
      v[d] = at < per_block && base + at < count ? __builtin_nontemporal_load(src + base + at)
                                                 : probe_f4{};
    }
#pragma unroll
    for (int d = 0; d < kReadProbeDepth; ++d) acc += v[d].x + v[d].y + v[d].z + v[d].w;
  }
  if (acc == 1234.5f) sink[0] = acc;
}

unsigned grid_for(size_t items) {
  const size_t blocks = (items + kThreads - 1) / kThreads;
  return (unsigned)(blocks < 65536 * 8 ? (blocks ? blocks : 1) : 65536 * 8);
}

bool float_dtype(int dtype) { return dtype == TMC_F16 || dtype == TMC_F32; }

}  // namespace
}  // namespace tmc

using namespace tmc;

#define TMC_DISPATCH_T(dtype, FN)                 \
  do {                                            \
    if ((dtype) == TMC_F32) {                     \
      typedef float T;                            \
      FN;                                         \
    } else {                                      \
      typedef half_t T;                           \
      FN;                                         \
    }                                             \
  } while (0)

namespace {

template <typename T>
void launch_norm_typed(bool add, const void* residual, const void* update, const void* w,
                       void* sum_out, void* norm_out, int64_t rows, int64_t width, float eps,
                       int threads, bool two_pass, hipStream_t stream) {
  const T* r = static_cast<const T*>(residual);
  const T* wt = static_cast<const T*>(w);
  T* n = static_cast<T*>(norm_out);
  if (add)
    launch_norm_threads<T, true>(r, static_cast<const T*>(update), wt, static_cast<T*>(sum_out),
                                 n, rows, width, eps, threads, two_pass, stream);
  else
    launch_norm_threads<T, false>(r, nullptr, wt, nullptr, n, rows, width, eps, threads, two_pass,
                                  stream);
}

int norm_entry(bool add, const void* residual, const void* update, const void* w, void* sum_out,
               void* norm_out, int dtype, int64_t rows, int64_t width, float epsilon,
               int threads, int variant, void* stream) {
  const char* what = add ? "Add+RMSNorm" : "RMSNorm";
  TMC_REQUIRE(residual && w && norm_out && (!add || (update && sum_out)),
              std::string(what) + ": null device pointer.");
  TMC_REQUIRE(float_dtype(dtype), std::string(what) + ": dtype must be fp16 or fp32.");
  TMC_REQUIRE(rows > 0 && width > 0 && width < (1LL << 31) && rows < (1LL << 31),
              std::string(what) + ": invalid shape.");
  TMC_REQUIRE(std::isfinite(epsilon) && epsilon > 0.0f,
              std::string(what) + ": epsilon must be finite and positive.");
  TMC_REQUIRE(variant == 0 || variant == 1,
              std::string(what) + ": variant must be 0 (default) or 1 (two-pass).");
  if (threads == 0) threads = kThreads;
  TMC_REQUIRE(threads == 64 || threads == 128 || threads == 256 || threads == 512 ||
                  threads == 1024,
              std::string(what) + ": threads must be 64, 128, 256, 512 or 1024.");
  const bool two_pass = variant == 1;
  if (dtype == TMC_F32)
    launch_norm_typed<float>(add, residual, update, w, sum_out, norm_out, rows, width, epsilon,
                             threads, two_pass, as_stream(stream));
  else
    launch_norm_typed<half_t>(add, residual, update, w, sum_out, norm_out, rows, width, epsilon,
                              threads, two_pass, as_stream(stream));
  return check_launch(add ? "add_rmsnorm kernel" : "rmsnorm kernel");
}

}  // namespace

extern "C" int tmc_rmsnorm(const void* x, const void* w, void* y, int dtype, int64_t rows,
                           int64_t width, float epsilon, void* stream) {
  return norm_entry(false, x, nullptr, w, nullptr, y, dtype, rows, width, epsilon, 0, 0, stream);
}

extern "C" int tmc_add_rmsnorm(const void* residual, const void* update, const void* w,
                               void* sum_out, void* norm_out, int dtype, int64_t rows,
                               int64_t width, float epsilon, void* stream) {
  return norm_entry(true, residual, update, w, sum_out, norm_out, dtype, rows, width, epsilon, 0,
                    0, stream);
}

extern "C" int tmc_add_rmsnorm_ex(const void* residual, const void* update, const void* w,
                                  void* sum_out, void* norm_out, int dtype, int64_t rows,
                                  int64_t width, float epsilon, int layout, void* stream) {
  TMC_REQUIRE(layout == 0 || layout == TMC_LAYOUT_Y_PACKED,
              "Add+RMSNorm: layout must be 0 or TMC_LAYOUT_Y_PACKED.");
  if (layout == 0)
    return norm_entry(update != nullptr, residual, update, w, sum_out, norm_out, dtype, rows,
                      width, epsilon, 0, 0, stream);
  TMC_REQUIRE(residual && w && norm_out && (!update || sum_out), "Add+RMSNorm: null device pointer.");
  TMC_REQUIRE(dtype == TMC_F16, "Add+RMSNorm: packed output needs fp16.");
  TMC_REQUIRE(rows > 0 && width > 0 && rows < (1LL << 31), "Add+RMSNorm: invalid shape.");
  TMC_REQUIRE(std::isfinite(epsilon) && epsilon > 0.0f,
              "Add+RMSNorm: epsilon must be finite and positive.");
  TMC_REQUIRE(aligned16(residual) && aligned16(w) && aligned16(norm_out) &&
                  (!update || (aligned16(update) && aligned16(sum_out))),
              "Add+RMSNorm: packed output needs 16-byte aligned operands.");
  const half_t* r = static_cast<const half_t*>(residual);
  const half_t* u = static_cast<const half_t*>(update);
  const half_t* g = static_cast<const half_t*>(w);
  half_t* s = static_cast<half_t*>(sum_out);
  half_t* n = static_cast<half_t*>(norm_out);
  const bool ok = update ? launch_norm_packed_out<true>(r, u, g, s, n, rows, width, epsilon,
                                                        as_stream(stream))
                         : launch_norm_packed_out<false>(r, nullptr, g, nullptr, n, rows, width,
                                                         epsilon, as_stream(stream));
  TMC_REQUIRE(ok, "Add+RMSNorm: packed output needs width % 8 == 0 and width <= 8192.");
  return check_launch("add_rmsnorm packed kernel");
}

extern "C" int tmc_rmsnorm_threads(const void* x, const void* w, void* y, int dtype,
                                   int64_t rows, int64_t width, float epsilon, int threads,
                                   int variant, void* stream) {
  return norm_entry(false, x, nullptr, w, nullptr, y, dtype, rows, width, epsilon, threads,
                    variant, stream);
}

extern "C" int tmc_add_rmsnorm_threads(const void* residual, const void* update, const void* w,
                                       void* sum_out, void* norm_out, int dtype, int64_t rows,
                                       int64_t width, float epsilon, int threads, int variant,
                                       void* stream) {
  return norm_entry(true, residual, update, w, sum_out, norm_out, dtype, rows, width, epsilon,
                    threads, variant, stream);
}

extern "C" int tmc_silu_mul(const void* gate, const void* up, void* out, int dtype, int64_t count,
                            void* stream) {
  TMC_REQUIRE(gate && up && out, "SiLU*Mul: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && count > 0, "SiLU*Mul: invalid dtype or count.");
  if (dtype == TMC_F16 && count % 8 == 0 && aligned16(gate) && aligned16(up) && aligned16(out)) {
    const size_t vectors = (size_t)count / 8;
    hipLaunchKernelGGL(silu_mul_h8_kernel, dim3(grid_for(vectors)), dim3(kThreads), 0,
                       as_stream(stream), static_cast<const h8*>(gate), static_cast<const h8*>(up),
                       static_cast<h8*>(out), vectors);
    return check_launch("silu_mul_h8_kernel");
  }
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((silu_mul_kernel<T>), dim3(grid_for(count)), dim3(kThreads), 0,
                                            as_stream(stream), static_cast<const T*>(gate),
                                            static_cast<const T*>(up), static_cast<T*>(out),
                                            (size_t)count));
  return check_launch("silu_mul_kernel");
}

extern "C" int tmc_add(const void* a, const void* b, void* out, int dtype, int64_t count,
                       void* stream) {
  TMC_REQUIRE(a && b && out, "Add: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && count > 0, "Add: invalid dtype or count.");
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((add_kernel<T>), dim3(grid_for(count)), dim3(kThreads), 0,
                                            as_stream(stream), static_cast<const T*>(a),
                                            static_cast<const T*>(b), static_cast<T*>(out),
                                            (size_t)count));
  return check_launch("add_kernel");
}

extern "C" int tmc_elementwise(int op, const void* a, const void* b, void* out, int dtype,
                               int64_t count, int threads, void* stream) {
  TMC_REQUIRE(op >= kEwAdd && op <= kEwSiluMul, "Elementwise: unknown operation.");
  TMC_REQUIRE(a && out && (op == kEwSilu || b), "Elementwise: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && count > 0, "Elementwise: invalid dtype or count.");
  TMC_REQUIRE(threads == 64 || threads == 128 || threads == 256,
              "Elementwise: threads must be 64, 128 or 256.");
  const unsigned blocks =
      (unsigned)std::min<size_t>(((size_t)count + threads - 1) / threads, 65536);
  switch (op) {
#define TMC_EW_CASE(OPC)                                                                   \
  case OPC:                                                                                \
    TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((elementwise_kernel<T, OPC>), dim3(blocks),   \
                                              dim3(threads), 0, as_stream(stream),         \
                                              static_cast<const T*>(a),                    \
                                              static_cast<const T*>(b), static_cast<T*>(out), \
                                              (size_t)count));                             \
    break;
    TMC_EW_CASE(kEwAdd)
    TMC_EW_CASE(kEwMul)
    TMC_EW_CASE(kEwSilu)
    TMC_EW_CASE(kEwSiluMul)
#undef TMC_EW_CASE
  }
  return check_launch("elementwise_kernel");
}

extern "C" int tmc_embedding(const int32_t* tokens, const void* table, void* out, int dtype,
                             int64_t rows, int64_t hidden, int64_t vocabulary, void* stream) {
  TMC_REQUIRE(tokens && table && out, "Embedding: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && rows > 0 && rows < 65536 && hidden > 0 && vocabulary > 0 &&
                  hidden < (1LL << 31) && vocabulary < (1LL << 31),
              "Embedding: invalid dtype or shape.");
  const dim3 grid((unsigned)((hidden + kThreads - 1) / kThreads), (unsigned)rows);
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((embedding_kernel<T>), grid, dim3(kThreads), 0,
                                            as_stream(stream), tokens, static_cast<const T*>(table),
                                            static_cast<T*>(out), (int)hidden, (int)vocabulary));
  return check_launch("embedding_kernel");
}

extern "C" int tmc_rope(const void* x, const float* cosine, const float* sine,
                        const int32_t* valid_length, void* out, int dtype, int64_t batch,
                        int64_t seq, int64_t heads, int64_t head_dim, int64_t capacity,
                        void* stream) {
  TMC_REQUIRE(x && cosine && sine && valid_length && out, "RoPE: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && batch > 0 && seq > 0 && heads > 0 && head_dim > 0 &&
                  head_dim % 2 == 0 && capacity >= seq,
              "RoPE: invalid dtype or shape.");
  const size_t items = (size_t)batch * heads * seq * (head_dim / 2);
  TMC_REQUIRE(items < (1ull << 40), "RoPE: too many elements.");
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((rope_kernel<T>), dim3((unsigned)((items + kThreads - 1) / kThreads)),
                                            dim3(kThreads), 0, as_stream(stream),
                                            static_cast<const T*>(x), cosine, sine, valid_length,
                                            static_cast<T*>(out), (int)batch, (int)seq, (int)heads,
                                            (int)head_dim, (int)capacity));
  return check_launch("rope_kernel");
}

extern "C" int tmc_serving_rope(const void* x, const float* cosine, const float* sine,
                                const int32_t* valid_lengths, const int32_t* active_count,
                                void* out, int dtype, int64_t max_batch, int64_t heads,
                                int64_t head_dim, int64_t capacity, void* stream) {
  TMC_REQUIRE(x && cosine && sine && valid_lengths && active_count && out,
              "Serving RoPE: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && max_batch > 0 && heads > 0 && head_dim > 0 &&
                  head_dim % 2 == 0 && capacity > 0,
              "Serving RoPE: invalid dtype or shape.");
  const size_t items = (size_t)max_batch * heads * (head_dim / 2);
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((serving_rope_kernel<T>), dim3((unsigned)((items + kThreads - 1) / kThreads)),
                                            dim3(kThreads), 0, as_stream(stream),
                                            static_cast<const T*>(x), cosine, sine, valid_lengths,
                                            active_count, static_cast<T*>(out), (int)max_batch,
                                            (int)heads, (int)head_dim, (int)capacity));
  return check_launch("serving_rope_kernel");
}

static int append_common(const void* input, const int32_t* valid_length, const int32_t* table,
                         void* cache, int dtype, int64_t batch, int64_t seq, int64_t heads,
                         int64_t head_dim, int64_t capacity, int64_t page_size, int head_major,
                         bool paged, void* stream) {
  TMC_REQUIRE(input && valid_length && cache && (!paged || table), "KV append: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && batch > 0 && seq > 0 && heads > 0 && head_dim > 0 &&
                  capacity >= seq && (!paged || (page_size > 0 && page_size <= capacity)),
              "KV append: invalid dtype or shape.");
  const size_t items = (size_t)batch * seq * heads * head_dim;
  const dim3 grid((unsigned)((items + kThreads - 1) / kThreads));
  if (paged) {
    TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((append_kernel<T, true>), grid, dim3(kThreads), 0,
                                              as_stream(stream), static_cast<const T*>(input),
                                              valid_length, table, static_cast<T*>(cache),
                                              (int)batch, (int)seq, (int)heads, (int)head_dim,
                                              (int)capacity, (int)page_size, head_major));
  } else {
    TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((append_kernel<T, false>), grid, dim3(kThreads), 0,
                                              as_stream(stream), static_cast<const T*>(input),
                                              valid_length, table, static_cast<T*>(cache),
                                              (int)batch, (int)seq, (int)heads, (int)head_dim,
                                              (int)capacity, 1, head_major));
  }
  return check_launch("append_kernel");
}

extern "C" int tmc_kv_append(const void* input, const int32_t* valid_length, void* cache,
                             int dtype, int64_t batch, int64_t seq, int64_t heads,
                             int64_t head_dim, int64_t capacity, int head_major, void* stream) {
  return append_common(input, valid_length, nullptr, cache, dtype, batch, seq, heads, head_dim,
                       capacity, 0, head_major, false, stream);
}

extern "C" int tmc_paged_kv_append(const void* input, const int32_t* valid_length,
                                   const int32_t* block_table, void* cache, int dtype,
                                   int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                                   int64_t capacity, int64_t page_size, int head_major,
                                   void* stream) {
  return append_common(input, valid_length, block_table, cache, dtype, batch, seq, heads,
                       head_dim, capacity, page_size, head_major, true, stream);
}

extern "C" int tmc_serving_kv_append(const void* input, const int32_t* valid_lengths,
                                     const int32_t* block_tables, const int32_t* active_count,
                                     void* cache, int dtype, int64_t max_batch, int64_t heads,
                                     int64_t head_dim, int64_t capacity, int64_t page_size,
                                     int head_major, void* stream) {
  TMC_REQUIRE(input && valid_lengths && block_tables && active_count && cache,
              "Serving KV append: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && max_batch > 0 && heads > 0 && head_dim > 0 && capacity > 0 &&
                  page_size > 0 && page_size <= capacity,
              "Serving KV append: invalid dtype or shape.");
  const size_t items = (size_t)max_batch * heads * head_dim;
  const dim3 grid((unsigned)((items + kThreads - 1) / kThreads));
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((serving_append_kernel<T>), grid, dim3(kThreads), 0,
                                            as_stream(stream), static_cast<const T*>(input),
                                            valid_lengths, block_tables, active_count,
                                            static_cast<T*>(cache), (int)max_batch, (int)heads,
                                            (int)head_dim, (int)capacity, (int)page_size,
                                            head_major));
  return check_launch("serving_append_kernel");
}

namespace {
int launch_rope_append(const void* qkv, const float* cosine, const float* sine,
                       const int32_t* valid_lengths, const int32_t* block_tables,
                       const int32_t* active_count, void* q_out, void* key_pool, void* value_pool,
                       int dtype, int64_t max_batch, int64_t q_heads, int64_t kv_heads,
                       int64_t head_dim, int64_t capacity, int64_t page_size, int64_t max_pages,
                       bool shared_table, const int32_t* row_table, int64_t table_rows,
                       void* stream) {
  TMC_REQUIRE(qkv && cosine && sine && valid_lengths && block_tables && active_count && q_out &&
                  key_pool && value_pool,
              "RoPE+append: null device pointer.");
  TMC_REQUIRE(float_dtype(dtype) && max_batch > 0 && max_batch < 65536 && q_heads > 0 &&
                  kv_heads > 0 && q_heads % kv_heads == 0 && head_dim > 0 && head_dim % 2 == 0 &&
                  head_dim <= 1024 && capacity > 0 && page_size > 0 && page_size <= capacity &&
                  max_pages == (capacity + page_size - 1) / page_size,
              "RoPE+append: invalid dtype or shape (max_pages must be "
              "ceil(capacity / page_size)).");
  const size_t items = (size_t)max_batch * (q_heads + 2 * kv_heads) * (head_dim / 2);
  TMC_REQUIRE(items < (1ull << 31), "RoPE+append: too many elements.");
  TMC_REQUIRE(!row_table || (table_rows >= 1 && table_rows < (1LL << 24)),
              "RoPE+append: a row table needs table_rows >= 1.");
  const int table_stride = shared_table && !row_table ? 0 : (int)max_pages;
  if (dtype == TMC_F16 && head_dim % 8 == 0 && aligned16(qkv) && aligned16(cosine) &&
      aligned16(sine) && aligned16(q_out) && aligned16(key_pool) && aligned16(value_pool)) {
    const size_t octs = items / 4;
    hipLaunchKernelGGL(decode_rope_append_h8_kernel,
                       dim3((unsigned)((octs + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       as_stream(stream), static_cast<const half_t*>(qkv), cosine, sine,
                       valid_lengths, block_tables, active_count, static_cast<half_t*>(q_out),
                       static_cast<half_t*>(key_pool), static_cast<half_t*>(value_pool),
                       (int)max_batch, (int)q_heads, (int)kv_heads, (int)head_dim, (int)capacity,
                       (int)page_size, table_stride, row_table, (int)table_rows);
    return check_launch("decode_rope_append_h8_kernel");
  }
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((decode_rope_append_kernel<T>),
                                            dim3((unsigned)((items + kThreads - 1) / kThreads)),
                                            dim3(kThreads), 0, as_stream(stream),
                                            static_cast<const T*>(qkv), cosine, sine,
                                            valid_lengths, block_tables, active_count,
                                            static_cast<T*>(q_out), static_cast<T*>(key_pool),
                                            static_cast<T*>(value_pool), (int)max_batch,
                                            (int)q_heads, (int)kv_heads, (int)head_dim,
                                            (int)capacity, (int)page_size, table_stride,
                                            row_table, (int)table_rows));
  return check_launch("decode_rope_append_kernel");
}
}  // namespace

extern "C" int tmc_decode_rope_append(const void* qkv, const float* cosine, const float* sine,
                                      const int32_t* valid_lengths, const int32_t* block_tables,
                                      const int32_t* active_count, void* q_out, void* key_pool,
                                      void* value_pool, int dtype, int64_t max_batch,
                                      int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                      int64_t capacity, int64_t page_size, int64_t max_pages,
                                      void* stream) {
  return launch_rope_append(qkv, cosine, sine, valid_lengths, block_tables, active_count, q_out,
                            key_pool, value_pool, dtype, max_batch, q_heads, kv_heads, head_dim,
                            capacity, page_size, max_pages, false, nullptr, 0, stream);
}

extern "C" int tmc_prefill_rope_append(const void* qkv, const float* cosine, const float* sine,
                                       const int32_t* valid_lengths, const int32_t* block_table,
                                       const int32_t* active_count, void* q_out, void* key_pool,
                                       void* value_pool, int dtype, int64_t rows, int64_t q_heads,
                                       int64_t kv_heads, int64_t head_dim, int64_t capacity,
                                       int64_t page_size, int64_t max_pages, void* stream) {
  return launch_rope_append(qkv, cosine, sine, valid_lengths, block_table, active_count, q_out,
                            key_pool, value_pool, dtype, rows, q_heads, kv_heads, head_dim,
                            capacity, page_size, max_pages, true, nullptr, 0, stream);
}

extern "C" int tmc_prefill_rope_append_rows(const void* qkv, const float* cosine, const float* sine,
                                            const int32_t* valid_lengths,
                                            const int32_t* block_tables, const int32_t* row_table,
                                            int64_t table_rows, const int32_t* active_count,
                                            void* q_out, void* key_pool, void* value_pool,
                                            int dtype, int64_t rows, int64_t q_heads,
                                            int64_t kv_heads, int64_t head_dim, int64_t capacity,
                                            int64_t page_size, int64_t max_pages, void* stream) {
  TMC_REQUIRE(row_table, "RoPE+append: null row table.");
  return launch_rope_append(qkv, cosine, sine, valid_lengths, block_tables, active_count, q_out,
                            key_pool, value_pool, dtype, rows, q_heads, kv_heads, head_dim,
                            capacity, page_size, max_pages, true, row_table, table_rows, stream);
}

namespace tmc {
namespace {
// emitLMHeadFinalArgmax (DecoderLLMMetalEmitter.cpp:730-753): one block per
// row folds the row's partial (value, index) slots, count from the
// workspace header, in the greedy-token order.
constexpr int kFinalArgmaxThreads = 256;
__global__ __launch_bounds__(kFinalArgmaxThreads) void final_argmax_kernel(
    void* workspace, int32_t* __restrict__ tokens, int rows, int cap) {
  const ArgmaxPartials in = argmax_partials(workspace, rows, cap);
  const int row = blockIdx.x;
  const int count = min(*in.count, cap);
  float best = -INFINITY;
  int selected = -1;
  for (int c = threadIdx.x; c < count; c += kFinalArgmaxThreads) {
    const float v = in.values[(size_t)row * cap + c];
    const int i = in.indices[(size_t)row * cap + c];
    if (argmax_better(v, i, best, selected)) {
      best = v;
      selected = i;
    }
  }
  argmax_wave(best, selected);
  __shared__ float wv[kFinalArgmaxThreads / kWave];
  __shared__ int wi[kFinalArgmaxThreads / kWave];
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    wv[wave] = best;
    wi[wave] = selected;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFinalArgmaxThreads / kWave; ++w)
      if (argmax_better(wv[w], wi[w], best, selected)) {
        best = wv[w];
        selected = wi[w];
      }
    tokens[row] = selected;
  }
}
}  // namespace
}  // namespace tmc

extern "C" size_t tmc_lm_head_argmax_workspace_bytes(int64_t rows, int64_t vocabulary) {
  if (rows <= 0 || vocabulary <= 0 || rows >= (1LL << 20) || vocabulary >= (1LL << 28)) return 0;
  return 256 + (size_t)rows * (size_t)vocabulary * (sizeof(float) + sizeof(int32_t));
}

extern "C" int tmc_lm_head_final_argmax(void* workspace, size_t workspace_bytes, int32_t* tokens,
                                        int64_t rows, int64_t vocabulary, void* stream) {
  TMC_REQUIRE(workspace && tokens, "LM head final argmax: null device pointer.");
  TMC_REQUIRE(rows > 0 && vocabulary > 0 && rows < (1LL << 20) && vocabulary < (1LL << 28),
              "LM head final argmax: invalid shape.");
  TMC_REQUIRE(workspace_bytes >= tmc_lm_head_argmax_workspace_bytes(rows, vocabulary),
              "LM head final argmax: workspace is smaller than "
              "tmc_lm_head_argmax_workspace_bytes().");
  hipLaunchKernelGGL(final_argmax_kernel, dim3((unsigned)rows), dim3(kFinalArgmaxThreads), 0,
                     as_stream(stream), workspace, tokens, (int)rows, (int)vocabulary);
  return check_launch("final_argmax_kernel");
}

extern "C" int tmc_argmax_f32(const float* logits, int32_t* tokens, int64_t rows,
                              int64_t vocabulary, void* stream) {
  TMC_REQUIRE(logits && tokens, "Argmax: null device pointer.");
  TMC_REQUIRE(rows > 0 && rows < (1LL << 31) && vocabulary > 0 && vocabulary < (1LL << 31),
              "Argmax: invalid shape.");
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(kArgmaxThreads), 0,
                     as_stream(stream), logits, tokens, (int)vocabulary);
  return check_launch("argmax_kernel");
}

namespace tmc {
namespace {
// Between two chained greedy-decode steps: row r's token becomes the next
// step's input token and the step's history entry, and its length grows by
// one (the position the next step appends).
__global__ __launch_bounds__(64) void decode_chain_kernel(const int32_t* __restrict__ next,
                                                          int32_t* __restrict__ tokens,
                                                          int32_t* __restrict__ lengths,
                                                          int32_t* __restrict__ history,
                                                          int rows) {
  for (int r = blockIdx.x * 64 + threadIdx.x; r < rows; r += gridDim.x * 64) {
    const int32_t token = next[r];
    tokens[r] = token;
    if (history) history[r] = token;
    if (lengths) lengths[r] += 1;
  }
}
}  // namespace
}  // namespace tmc

extern "C" int tmc_decode_chain(const int32_t* next_tokens, int32_t* tokens, int32_t* lengths,
                                int32_t* history, int64_t rows, void* stream) {
  TMC_REQUIRE(next_tokens && tokens, "Decode chain: null device pointer.");
  TMC_REQUIRE(rows > 0 && rows <= (1LL << 20), "Decode chain: rows must be in [1, 2^20].");
  const unsigned blocks = (unsigned)std::min<int64_t>((rows + 63) / 64, 64);
  hipLaunchKernelGGL(tmc::decode_chain_kernel, dim3(blocks), dim3(64), 0, as_stream(stream),
                     next_tokens, tokens, lengths, history, (int)rows);
  return check_launch("decode_chain_kernel");
}

extern "C" int tmc_fill_normal(void* ptr, int dtype, int64_t count, uint64_t seed, float mean,
                               float std, void* stream) {
  TMC_REQUIRE(ptr && count > 0 && float_dtype(dtype), "Fill: invalid arguments.");
  TMC_DISPATCH_T(dtype, hipLaunchKernelGGL((fill_normal_kernel<T>), dim3(grid_for(count)), dim3(kThreads), 0,
                                            as_stream(stream), static_cast<T*>(ptr), (size_t)count,
                                            seed, mean, std));
  return check_launch("fill_normal_kernel");
}

namespace tmc {
namespace {

// blockIdx.y = page index i; threads copy 16-byte units of one page.
__global__ __launch_bounds__(256) void copy_pages_kernel(const uint4* __restrict__ src,
                                                         uint4* __restrict__ dst,
                                                         const int32_t* __restrict__ pages,
                                                         size_t units, int scatter) {
  const size_t i = blockIdx.y;
  const size_t page = (size_t)pages[i];
  const size_t from = scatter ? i : page, to = scatter ? page : i;
  for (size_t u = (size_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (size_t)gridDim.x * 256)
    dst[to * units + u] = src[from * units + u];
}

}  // namespace
}  // namespace tmc

extern "C" int tmc_host_alloc(size_t bytes, void** out) {
  TMC_REQUIRE(out && bytes > 0, "Host alloc: invalid arguments.");
  *out = nullptr;
  // Mapped: kernels read and write it directly (ROCm gives it the same
  // address on the device).
  const hipError_t rc = hipHostMalloc(out, bytes, hipHostMallocMapped);
  TMC_REQUIRE(rc == hipSuccess, std::string("Host alloc: hipHostMalloc failed: ") +
                                    hipGetErrorString(rc));
  return 0;
}

extern "C" void tmc_host_free(void* ptr) {
  if (ptr) (void)hipHostFree(ptr);
}

extern "C" int tmc_copy_pages(const void* src, void* dst, const int32_t* pages, int64_t count,
                              int64_t page_bytes, int scatter, void* stream) {
  TMC_REQUIRE(src && dst && pages, "Copy pages: null pointer.");
  TMC_REQUIRE(count > 0 && count < 65536 && page_bytes > 0 && page_bytes % 16 == 0,
              "Copy pages: count must be in [1, 65535] and page_bytes a multiple of 16.");
  TMC_REQUIRE(aligned16(src) && aligned16(dst), "Copy pages: buffers must be 16-byte aligned.");
  const size_t units = (size_t)page_bytes / 16;
  const dim3 grid((unsigned)std::min<size_t>((units + 255) / 256, 64), (unsigned)count);
  hipLaunchKernelGGL(copy_pages_kernel, grid, dim3(256), 0, as_stream(stream),
                     static_cast<const uint4*>(src), static_cast<uint4*>(dst), pages, units,
                     scatter);
  return check_launch("copy_pages_kernel");
}

extern "C" int tmc_read_probe(const void* src, size_t bytes, void* sink, void* stream) {
  TMC_REQUIRE(src && sink && bytes > 0 && bytes % 16 == 0 && aligned16(src),
              "Read probe: src must be 16-byte aligned and size a multiple of 16.");
  const size_t count = bytes / 16;
  const size_t per_block = (count + kReadProbeBlocks - 1) / kReadProbeBlocks;
  hipLaunchKernelGGL(read_probe_kernel, dim3(kReadProbeBlocks), dim3(256), 0, as_stream(stream),
                     static_cast<const probe_f4*>(src), static_cast<float*>(sink), count, per_block);
  return check_launch("read_probe_kernel");
}

extern "C" int tmc_copy_bytes(const void* src, void* dst, size_t bytes, void* stream) {
  TMC_REQUIRE(src && dst && bytes > 0 && bytes % 16 == 0 && aligned16(src) && aligned16(dst),
              "Copy: pointers must be 16-byte aligned and size a multiple of 16.");
  const size_t count = bytes / 16;
  hipLaunchKernelGGL(copy_kernel, dim3(grid_for(count)), dim3(kThreads), 0, as_stream(stream),
                     static_cast<const uint4*>(src), static_cast<uint4*>(dst), count);
  return check_launch("copy_kernel");
}
