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
// Wave layout for head dim D: RL = D/8 lanes hold one position's 16-byte
// slices, so one 16-byte load instruction covers NR = 64/RL consecutive
// positions (one contiguous 1 KiB run for D = 128 inside a 16-token page).
// A wave tile is J = 4 such loads (TILE = 4*NR positions); each lane keeps
// its own 4 positions' softmax terms and its 8 output columns, and rows are
// folded together only once per split (cross-row shuffles), then the 4 waves
// of the block merge through LDS.  Splits merge in attn_combine_kernel.
#include "tmc_abi.hpp"
#include "tmc_device.hpp"

namespace tmc {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTilesPerWave = 4;

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
  float scale_log2;       // (1/sqrt(D)) * log2(e)
};

template <int D> constexpr int chunk_positions() {
  return kWaves * kTilesPerWave * 4 * (kWave / (D / 8));
}

template <bool PAGED>
__device__ __forceinline__ int valid_length(const AttnParams& p, int b) {
  return PAGED ? p.valid[b] : p.valid[0];
}

// True when a page needed by [0, valid) is negative (the reference kernel
// returns before writing in that case).  Block-uniform result.
__device__ __forceinline__ bool has_bad_page(const AttnParams& p, int b, int valid) {
  const int pages = (valid + p.page_size - 1) / p.page_size;
  int bad = 0;
  for (int lp = threadIdx.x; lp < pages; lp += blockDim.x)
    bad |= p.tables[(size_t)b * p.max_pages + lp] < 0;
  return __syncthreads_or(bad) != 0;
}

template <int D, int GROUP, bool PAGED>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(AttnParams p) {
  constexpr int RL = D / 8;
  constexpr int NR = kWave / RL;
  constexpr int J = 4;
  constexpr int TILE = NR * J;
  constexpr int CHUNK = chunk_positions<D>();
  __shared__ float s_m[kWaves][GROUP];
  __shared__ float s_l[kWaves][GROUP];
  __shared__ float s_o[kWaves][GROUP][D];

  const int b = blockIdx.z, kvh = blockIdx.y, split = blockIdx.x;
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
  const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  const size_t contiguous_base = ((size_t)b * p.kv_heads + kvh) * (size_t)p.capacity * D;

  for (int tile = wave;; tile += kWaves) {
    const int p0 = begin + tile * TILE;
    if (p0 >= end) break;  // wave-uniform
    h8 kv[J], vv[J];
    bool ok[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int pos = p0 + r + NR * j;
      ok[j] = pos < end;
      size_t off = 0;
      if constexpr (PAGED) {
        const int page = ok[j] ? p.tables[(size_t)b * p.max_pages + pos / p.page_size] : -1;
        ok[j] = ok[j] && page >= 0;
        off = (size_t)page * p.page_stride + (size_t)kvh * p.head_stride +
              (size_t)(pos % p.page_size) * D + 8 * c;
      } else {
        off = contiguous_base + (size_t)pos * D + 8 * c;
      }
      kv[j] = ok[j] ? load_h8(p.k + off) : zero;
      vv[j] = ok[j] ? load_h8(p.v + off) : zero;
    }
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
      float s[J];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const float dot = group_sum<RL>(dot8(qv[g], kv[j], 0.0f));
        s[j] = ok[j] ? dot * p.scale_log2 : -INFINITY;
      }
      float tile_max = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      tile_max = cross_max<RL>(tile_max);
      const float next = fmaxf(m[g], tile_max);
      const float alpha = next == -INFINITY ? 1.0f : fast_exp2(m[g] - next);
      float psum = 0.0f;
#pragma unroll
      for (int t = 0; t < 8; ++t) o[g][t] *= alpha;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const float pj = ok[j] ? fast_exp2(s[j] - next) : 0.0f;
        psum += pj;
#pragma unroll
        for (int t = 0; t < 8; ++t) o[g][t] += pj * (float)vv[j][t];
      }
      l[g] = l[g] * alpha + psum;
      m[g] = next;
    }
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

  const bool single = nsplit == 1;
  if (PAGED && single && has_bad_page(p, b, valid)) return;
  for (int idx = threadIdx.x; idx < GROUP * D; idx += kThreads) {
    const int g = idx / D, d = idx % D;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][g]);
    float lsum = 0.0f, osum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float scale = s_m[w][g] == -INFINITY ? 0.0f : fast_exp2(s_m[w][g] - mx);
      lsum += scale * s_l[w][g];
      osum += scale * s_o[w][g][d];
    }
    const int qh = kvh * GROUP + g;
    if (single) {
      p.out[((size_t)b * p.q_heads + qh) * D + d] = (half_t)(osum / lsum);
    } else {
      float* slot = p.ws + (((size_t)b * p.q_heads + qh) * p.max_splits + split) * (D + 2);
      slot[d] = osum;
      if (d == 0) {
        slot[D] = mx;
        slot[D + 1] = lsum;
      }
    }
  }
}

template <int D, bool PAGED>
__global__ __launch_bounds__(D) void attn_combine_kernel(AttnParams p) {
  constexpr int CHUNK = chunk_positions<D>();
  const int qh = blockIdx.x, b = blockIdx.y;
  if (PAGED && p.active && b >= p.active[0]) return;
  const int valid = valid_length<PAGED>(p, b);
  if (valid < 1 || valid > p.capacity) return;
  const int nsplit = (valid + CHUNK - 1) / CHUNK;
  if (nsplit <= 1) return;
  if (PAGED && has_bad_page(p, b, valid)) return;
  const int d = threadIdx.x;
  const float* base = p.ws + ((size_t)b * p.q_heads + qh) * p.max_splits * (D + 2);
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, base[(size_t)s * (D + 2) + D]);
  float lsum = 0.0f, osum = 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const float* slot = base + (size_t)s * (D + 2);
    const float scale = slot[D] == -INFINITY ? 0.0f : fast_exp2(slot[D] - mx);
    lsum += scale * slot[D + 1];
    osum += scale * slot[d];
  }
  p.out[((size_t)b * p.q_heads + qh) * D + d] = (half_t)(osum / lsum);
}

template <int D, bool PAGED>
int launch_attention(const AttnParams& p, int batch, hipStream_t stream) {
  const int group = p.q_heads / p.kv_heads;
  const dim3 grid((unsigned)p.max_splits, (unsigned)p.kv_heads, (unsigned)batch);
  switch (group) {
  case 1: hipLaunchKernelGGL((attn_partial_kernel<D, 1, PAGED>), grid, dim3(kThreads), 0, stream, p); break;
  case 2: hipLaunchKernelGGL((attn_partial_kernel<D, 2, PAGED>), grid, dim3(kThreads), 0, stream, p); break;
  case 4: hipLaunchKernelGGL((attn_partial_kernel<D, 4, PAGED>), grid, dim3(kThreads), 0, stream, p); break;
  case 8: hipLaunchKernelGGL((attn_partial_kernel<D, 8, PAGED>), grid, dim3(kThreads), 0, stream, p); break;
  default: return fail("Attention: q_heads / kv_heads must be 1, 2, 4 or 8.");
  }
  if (check_launch("attn_partial_kernel")) return 1;
  if (p.max_splits > 1) {
    hipLaunchKernelGGL((attn_combine_kernel<D, PAGED>), dim3((unsigned)p.q_heads, (unsigned)batch),
                       dim3(D), 0, stream, p);
    return check_launch("attn_combine_kernel");
  }
  return 0;
}

int chunk_for(int64_t head_dim) {
  switch (head_dim) {
  case 16: return chunk_positions<16>();
  case 32: return chunk_positions<32>();
  case 64: return chunk_positions<64>();
  case 128: return chunk_positions<128>();
  default: return 0;
  }
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
  TMC_REQUIRE(chunk_for(head_dim) > 0, "Attention: head_dim must be 16, 32, 64 or 128.");
  TMC_REQUIRE(batch > 0 && batch < 65536 && q_heads > 0 && kv_heads > 0 && kv_heads < 65536 &&
                  q_heads % kv_heads == 0 && capacity > 0 && capacity < (1LL << 30),
              "Attention: invalid batch, head counts or capacity.");
  TMC_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v), "Attention: q, K and V must be 16-byte aligned.");
  return 0;
}

}  // namespace
}  // namespace tmc

using namespace tmc;

extern "C" size_t tmc_attention_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_dim,
                                                int64_t capacity) {
  const int chunk = chunk_for(head_dim);
  if (chunk <= 0 || batch <= 0 || q_heads <= 0 || capacity <= 0) return 0;
  const int64_t splits = (capacity + chunk - 1) / chunk;
  if (splits <= 1) return 0;
  return (size_t)batch * q_heads * splits * (head_dim + 2) * sizeof(float);
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
  const size_t need = tmc_attention_workspace_bytes(batch, q_heads, head_dim, capacity);
  TMC_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "Attention: workspace is smaller than tmc_attention_workspace_bytes().");
  AttnParams p{};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(key_cache);
  p.v = static_cast<const half_t*>(value_cache);
  p.out = static_cast<half_t*>(out);
  p.ws = static_cast<float*>(workspace);
  p.valid = valid_length;
  p.q_heads = (int)q_heads;
  p.kv_heads = (int)kv_heads;
  p.capacity = (int)capacity;
  p.page_size = 1;
  const int chunk = chunk_for(head_dim);
  p.max_splits = (int)((capacity + chunk - 1) / chunk);
  p.scale_log2 = (float)(1.0 / std::sqrt((double)head_dim)) * 1.4426950408889634f;
  return dispatch_attention<false>(p, (int)batch, (int)head_dim, as_stream(stream));
}

extern "C" int tmc_paged_decode_attention(const void* q, const void* key_pool,
                                          const void* value_pool, const int32_t* valid_lengths,
                                          const int32_t* block_tables,
                                          const int32_t* active_count, void* out, int dtype,
                                          int64_t max_batch, int64_t q_heads, int64_t kv_heads,
                                          int64_t head_dim, int64_t page_size, int64_t max_pages,
                                          int64_t page_stride, int64_t head_stride,
                                          void* workspace, size_t workspace_bytes,
                                          void* stream) {
  const int64_t capacity = page_size * max_pages;
  if (common_checks(q, key_pool, value_pool, out, dtype, max_batch, q_heads, kv_heads, head_dim,
                    capacity))
    return 1;
  TMC_REQUIRE(valid_lengths && block_tables, "Paged attention: null lengths or block tables.");
  TMC_REQUIRE(page_size > 0 && max_pages > 0 && page_stride > 0 && head_stride >= 0 &&
                  (page_stride % 8) == 0 && (head_stride % 8) == 0,
              "Paged attention: invalid page geometry (strides must be multiples of 8 elements).");
  const size_t need = tmc_attention_workspace_bytes(max_batch, q_heads, head_dim, capacity);
  TMC_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "Paged attention: workspace is smaller than tmc_attention_workspace_bytes().");
  AttnParams p{};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(key_pool);
  p.v = static_cast<const half_t*>(value_pool);
  p.out = static_cast<half_t*>(out);
  p.ws = static_cast<float*>(workspace);
  p.valid = valid_lengths;
  p.tables = block_tables;
  p.active = active_count;
  p.page_stride = (long)page_stride;
  p.head_stride = (long)head_stride;
  p.q_heads = (int)q_heads;
  p.kv_heads = (int)kv_heads;
  p.capacity = (int)capacity;
  p.page_size = (int)page_size;
  p.max_pages = (int)max_pages;
  const int chunk = chunk_for(head_dim);
  p.max_splits = (int)((capacity + chunk - 1) / chunk);
  p.scale_log2 = (float)(1.0 / std::sqrt((double)head_dim)) * 1.4426950408889634f;
  return dispatch_attention<true>(p, (int)max_batch, (int)head_dim, as_stream(stream));
}
