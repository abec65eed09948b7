// Runtime objects of the C ABI: the HIP counterpart of MetalRuntime,
// MetalBuffer, PreparedExecution and PreparedSequence
// (/root/reference/src/backend/metal/MetalRuntime.hpp:56-208, .mm:140-781).
//
//  * Buffers are hipMalloc allocations with the reference's host conversion
//    rules (fp16 ties away from zero, bf16 RNE, int32 truncation) and its
//    NaN / zero fill for fresh buffers.
//  * Kernels are resolved from a static table keyed "name?k=v&...", which
//    replaces runtime MSL compilation plus pipeline reflection: each entry
//    declares its binding types and writability and launches one of the
//    typed gfx950 entry points.
//  * A prepared execution owns its bindings, constants and any workspace.
//  * A sequence is captured once into a HIP graph and replayed with a single
//    hipGraphLaunch (the counterpart of one Metal command buffer); one that
//    holds a library call kept out of graphs (the prompt GEMM) replays its
//    steps eagerly on the same stream instead.
#include "tmc_abi.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace tmc {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& message) { g_error = message; }
void clear_error() { g_error.clear(); }

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return 0;
  set_error(std::string(what) + ": launch failed: " + hipGetErrorString(err));
  return 1;
}

namespace {

// ------------------------------------------------------------------ host conversions
// The upload/readback rules of MetalRuntime.mm:42-104: fp32 -> fp16 rounds
// to nearest with ties away from zero (NaN -> 0x7e00 with its sign, overflow
// -> inf), fp32 -> bf16 rounds to nearest even on the raw bits, int32 is a
// truncating cast.  The fp16 rounding is done arithmetically: the magnitude
// is scaled (exactly, in double) so that one fp16 step is 1, rounded with
// floor(x + 0.5), and the step count is reassembled into the bit fields.
uint16_t f16_bits(float value) {
  const uint16_t sign = std::signbit(value) ? 0x8000u : 0u;
  if (std::isnan(value)) return sign | 0x7e00u;
  const double magnitude = std::fabs((double)value);
  // 65520 is halfway between the largest fp16 (65504) and the next step.
  if (magnitude >= 65520.0) return sign | 0x7c00u;
  if (magnitude < 0x1p-14) {
    // subnormal steps of 2^-24; 1024 steps carry into the smallest normal
    return sign | (uint16_t)std::floor(std::ldexp(magnitude, 24) + 0.5);
  }
  int binary_exponent;
  std::frexp(magnitude, &binary_exponent);  // magnitude in [2^(e-1), 2^e)
  int exponent = binary_exponent - 1;
  double steps = std::floor(std::ldexp(magnitude, 10 - exponent) + 0.5);  // [1024, 2048]
  if (steps == 2048.0) {
    steps = 1024.0;
    ++exponent;
  }
  return sign | (uint16_t)((exponent + 15) << 10) | (uint16_t)(steps - 1024.0);
}

float f16_value(uint16_t half) {
  const unsigned exponent = (half >> 10) & 0x1fu, mantissa = half & 0x3ffu;
  float magnitude;
  if (exponent == 31) {
    const uint32_t bits = 0x7f800000u | (mantissa << 13);  // inf, or NaN keeping its payload
    std::memcpy(&magnitude, &bits, sizeof magnitude);
  } else if (exponent == 0) {
    magnitude = (float)std::ldexp((double)mantissa, -24);
  } else {
    magnitude = (float)std::ldexp((double)(1024u + mantissa), (int)exponent - 25);
  }
  return std::copysign(magnitude, (half & 0x8000u) ? -1.0f : 1.0f);
}

uint16_t bf16_bits(float value) {
  uint32_t bits;
  std::memcpy(&bits, &value, sizeof bits);
  uint32_t upper = bits >> 16;
  const uint32_t lower = bits & 0xffffu;
  if (lower > 0x8000u || (lower == 0x8000u && (upper & 1u))) ++upper;  // nearest, ties to even
  return (uint16_t)upper;
}

float bf16_value(uint16_t v) {
  const uint32_t bits = (uint32_t)v << 16;
  float out;
  std::memcpy(&out, &bits, sizeof out);
  return out;
}

size_t element_bytes(int dtype) { return dtype == TMC_F16 || dtype == TMC_BF16 ? 2 : 4; }
bool valid_dtype(int dtype) { return dtype >= TMC_F16 && dtype <= TMC_I32; }

void encode_into(const float* src, size_t count, int dtype, void* dst) {
  for (size_t i = 0; i < count; ++i) {
    switch (dtype) {
    case TMC_F16: static_cast<uint16_t*>(dst)[i] = f16_bits(src[i]); break;
    case TMC_BF16: static_cast<uint16_t*>(dst)[i] = bf16_bits(src[i]); break;
    case TMC_I32: static_cast<int32_t*>(dst)[i] = (int32_t)src[i]; break;
    default: static_cast<float*>(dst)[i] = src[i]; break;
    }
  }
}

void decode_into(const void* src, size_t count, int dtype, float* dst) {
  for (size_t i = 0; i < count; ++i) {
    switch (dtype) {
    case TMC_F16: dst[i] = f16_value(static_cast<const uint16_t*>(src)[i]); break;
    case TMC_BF16: dst[i] = bf16_value(static_cast<const uint16_t*>(src)[i]); break;
    case TMC_I32: dst[i] = (float)static_cast<const int32_t*>(src)[i]; break;
    default: dst[i] = static_cast<const float*>(src)[i]; break;
    }
  }
}

std::vector<uint8_t> encode(const float* src, size_t count, int dtype) {
  std::vector<uint8_t> out(count * element_bytes(dtype));
  encode_into(src, count, dtype, out.data());
  return out;
}

int hip_ok(hipError_t err, const char* what) {
  if (err == hipSuccess) return 0;
  set_error(std::string(what) + ": " + hipGetErrorString(err));
  return 1;
}

// Fill with the reference sentinel of each dtype (MetalRuntime.mm:200-215,
// :548-556).  `fresh` selects createBuffer's int fill (0) over run()'s
// INT32_MIN.
int fill_sentinel(void* ptr, size_t count, int dtype, bool fresh, hipStream_t stream) {
  hipError_t err;
  switch (dtype) {
  case TMC_F32: err = hipMemsetD32Async(ptr, 0x7fc00000, count, stream); break;
  case TMC_F16: err = hipMemsetD16Async(ptr, 0x7e00, count, stream); break;
  case TMC_BF16: err = hipMemsetD16Async(ptr, 0x7fc0, count, stream); break;
  default: err = hipMemsetD32Async(ptr, fresh ? 0 : (int)0x80000000u, count, stream); break;
  }
  return hip_ok(err, "sentinel fill");
}

}  // namespace
}  // namespace tmc

using namespace tmc;

// ====================================================================== objects
struct tmc_runtime {
  bool available = false;
  std::string device_name;
  std::string init_error;
  hipStream_t stream = nullptr;
  hipDeviceProp_t props{};
  int fail_next = 0;
  // Pinned staging of tmc_buf_write_raw_async and tmc_buf_write_sparse_async:
  // copies and scatter launches are appended at `staged`; once `staged_done`
  // (recorded after the last queued one) has completed, every staged byte has
  // reached the device and the area is reused from the start.
  char* staging = nullptr;
  char* staging_device = nullptr;  // the same pinned area as the device addresses it
  size_t staged = 0;
  hipEvent_t staged_done = nullptr;
};

struct tmc_buffer {
  tmc_runtime* rt = nullptr;
  void* ptr = nullptr;
  size_t count = 0;
  int dtype = TMC_F32;
  bool owned = true;
};

namespace {

struct LaunchContext {
  std::vector<void*> ptrs;     // inputs then outputs, device addresses
  std::vector<size_t> counts;  // their element counts
  std::vector<uint32_t> constants;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  hipStream_t stream = nullptr;
};

using Params = std::map<std::string, std::string>;

struct KernelSpec {
  std::vector<int> inputs;
  std::vector<int> outputs;
  size_t groups = 1;
  size_t threads = 256;
  size_t workspace_bytes = 0;
  // Minimum element count of every binding (inputs, then outputs) that the
  // launch reads or writes at this specialization; 0 = not checked (page
  // pools, whose extent the block tables decide).
  std::vector<size_t> counts;
  std::function<int(const LaunchContext&)> launch;
  // false: the launch calls a library that is not recorded into a graph
  // (the prompt GEMM); a sequence holding such a step replays eagerly.
  bool capturable = true;
};

}  // namespace

struct tmc_kernel {
  std::string key;
  KernelSpec spec;
};

// A prepared execution keeps its own copy of the kernel entry, so releasing
// the resolved kernel does not invalidate it (PreparedExecution owns its
// pipeline, MetalRuntime.hpp:101-102).
struct tmc_exec {
  tmc_runtime* rt = nullptr;
  KernelSpec spec;
  std::vector<tmc_buffer*> outputs;
  LaunchContext ctx;
};

struct tmc_seq {
  tmc_runtime* rt = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  // Eager replay (a step is not capturable): the steps' launches in order.
  std::vector<std::pair<std::function<int(const LaunchContext&)>, LaunchContext>> eager;
};

namespace {

int64_t param_int(const Params& p, const char* name, int64_t fallback = -1) {
  const auto it = p.find(name);
  if (it == p.end()) return fallback;
  return std::strtoll(it->second.c_str(), nullptr, 10);
}

double param_double(const Params& p, const char* name, double fallback) {
  const auto it = p.find(name);
  if (it == p.end()) return fallback;
  return std::strtod(it->second.c_str(), nullptr);
}

int param_dtype(const Params& p, const char* name, int fallback) {
  const auto it = p.find(name);
  if (it == p.end()) return fallback;
  const std::string& v = it->second;
  if (v == "f16" || v == "fp16") return TMC_F16;
  if (v == "f32" || v == "fp32") return TMC_F32;
  if (v == "bf16") return TMC_BF16;
  if (v == "i32" || v == "int32") return TMC_I32;
  return -1;
}

bool parse_key(const std::string& key, std::string& name, Params& params) {
  const auto q = key.find('?');
  name = key.substr(0, q);
  if (q == std::string::npos) return !name.empty();
  size_t pos = q + 1;
  while (pos < key.size()) {
    auto amp = key.find('&', pos);
    if (amp == std::string::npos) amp = key.size();
    const auto item = key.substr(pos, amp - pos);
    const auto eq = item.find('=');
    if (eq == std::string::npos || eq == 0) return false;
    params[item.substr(0, eq)] = item.substr(eq + 1);
    pos = amp + 1;
  }
  return !name.empty();
}

// Activation layouts of the packed GEMM keys: x_layout / y_layout =
// row_major (default) | packed.
bool layout_param(const Params& p, int& layout) {
  layout = 0;
  for (const auto& [field, bit] :
       {std::pair<const char*, int>{"x_layout", TMC_LAYOUT_X_PACKED}, {"y_layout", TMC_LAYOUT_Y_PACKED}}) {
    const auto it = p.find(field);
    if (it == p.end() || it->second == "row_major") continue;
    if (it->second != "packed") return false;
    layout |= bit;
  }
  return true;
}

// Optional GEMV launch configuration in a key: algorithm (0 auto, 1 dot,
// 2 MFMA, 3 MFMA row tiles, 4 linear baseline, 5 persistent dot at batch 1),
// rows_per_wave, unroll, k_split.  Validated when the kernel launches.
bool gemv_config_param(const Params& p, tmc_gemv_config& cfg) {
  cfg.algorithm = (int)param_int(p, "algorithm", 0);
  cfg.rows_per_wave = (int)param_int(p, "rows_per_wave", 1);
  cfg.unroll = (int)param_int(p, "unroll", 1);
  cfg.k_split = (int)param_int(p, "k_split", 1);
  return cfg.algorithm >= 0 && cfg.algorithm <= 5;
}

#define NEED(cond, msg)          \
  do {                           \
    if (!(cond)) {               \
      set_error(msg);            \
      return false;              \
    }                            \
  } while (0)

// Build the kernel table entry for `name` with its specialization.
bool make_spec(const std::string& name, const Params& p, KernelSpec& s) {
  const int dt = param_dtype(p, "dtype", TMC_F16);
  NEED(dt >= 0, "Unknown dtype in kernel key.");
  if (name == "decode_gemv") {
    const int64_t b = param_int(p, "batch"), k = param_int(p, "in"), n = param_int(p, "out");
    const int od = param_dtype(p, "out_dtype", TMC_F16);
    NEED(b > 0 && k > 0 && n > 0 && (od == TMC_F16 || od == TMC_F32) && dt == TMC_F16,
         "decode_gemv needs batch, in, out > 0, dtype=f16 and out_dtype f16|f32.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    s.inputs = {TMC_F16, TMC_F16};
    s.outputs = {od};
    s.counts = {(size_t)(b * k), (size_t)(n * k), (size_t)(b * n)};
    s.groups = (size_t)((n + 3) / 4);
    s.launch = [=](const LaunchContext& c) {
      return tmc_gemv_f16_config(c.ptrs[0], c.ptrs[1], c.ptrs[2], od, b, k, n, &cfg, c.stream);
    };
    return true;
  }
  if (name == "gemv_residual") {
    // Batch-1 GEMV with the residual add in its epilogue: inputs x, weight,
    // residual; output h(residual + h(W x)).
    const int64_t k = param_int(p, "in"), n = param_int(p, "out");
    NEED(param_int(p, "batch", 1) == 1 && k > 0 && n > 0 && dt == TMC_F16,
         "gemv_residual needs batch=1, in, out > 0 and dtype=f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    s.inputs = {TMC_F16, TMC_F16, TMC_F16};
    s.outputs = {TMC_F16};
    s.counts = {(size_t)k, (size_t)(n * k), (size_t)n, (size_t)n};
    s.groups = (size_t)((n + 3) / 4);
    s.launch = [=](const LaunchContext& c) {
      return tmc_gemv_residual_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], 1, k, n, &cfg,
                                   c.stream);
    };
    return true;
  }
  if (name == "add_rmsnorm_gemv" || name == "rmsnorm_gemv" || name == "add_rmsnorm_gate_up_silu" ||
      name == "rmsnorm_gate_up_silu") {
    // Batch-1 norm folded into the GEMV: inputs residual[, update], gamma,
    // weight(s); outputs [sum,] y.
    const bool add = name.rfind("add_", 0) == 0;
    const bool gated = name.find("gate_up") != std::string::npos;
    const int64_t k = param_int(p, "in"), n = param_int(p, "out");
    const float eps = (float)param_double(p, "eps", 1e-5);
    const int od = gated ? TMC_F16 : param_dtype(p, "out_dtype", TMC_F16);
    NEED(param_int(p, "batch", 1) == 1 && k > 0 && n > 0 && dt == TMC_F16 &&
             (od == TMC_F16 || od == TMC_F32),
         "fused norm kernels need batch=1, in, out > 0, f16 and out_dtype f16|f32.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    s.inputs = add ? std::vector<int>{TMC_F16, TMC_F16, TMC_F16} : std::vector<int>{TMC_F16, TMC_F16};
    s.inputs.push_back(TMC_F16);
    if (gated) s.inputs.push_back(TMC_F16);
    s.outputs = add ? std::vector<int>{TMC_F16, od} : std::vector<int>{od};
    s.counts = {(size_t)k};
    if (add) s.counts.push_back((size_t)k);
    s.counts.push_back((size_t)k);
    s.counts.push_back((size_t)(n * k));
    if (gated) s.counts.push_back((size_t)(n * k));
    if (add) s.counts.push_back((size_t)k);
    s.counts.push_back((size_t)n);
    s.groups = (size_t)((n + 7) / 8);
    s.launch = [=](const LaunchContext& c) {
      const int i = add ? 1 : 0;  // index shift past the update binding
      const void* update = add ? c.ptrs[1] : nullptr;
      const void* gamma = c.ptrs[1 + i];
      const void* w0 = c.ptrs[2 + i];
      const void* w1 = gated ? c.ptrs[3 + i] : nullptr;
      const int out0 = gated ? 4 + i : 3 + i;
      void* sum = add ? c.ptrs[out0] : nullptr;
      void* y = c.ptrs[add ? out0 + 1 : out0];
      if (gated)
        return tmc_add_rmsnorm_gate_up_silu_f16(c.ptrs[0], update, gamma, w0, w1, sum, y, 1, k, n,
                                                eps, &cfg, c.stream);
      return tmc_add_rmsnorm_gemv_f16(c.ptrs[0], update, gamma, w0, sum, y, od, 1, k, n, eps, &cfg,
                                      c.stream);
    };
    return true;
  }
  if (name == "pack_weights") {
    const int64_t n = param_int(p, "out"), k = param_int(p, "in");
    NEED(n > 0 && k > 0 && dt == TMC_F16, "pack_weights needs out, in > 0 and f16.");
    s.inputs = {TMC_F16};
    s.outputs = {TMC_F16};
    s.counts = {(size_t)(n * k), (size_t)tmc_packed_weight_elements(n, k)};
    s.groups = (size_t)((tmc_packed_weight_elements(n, k) / 8 + 255) / 256);
    s.launch = [=](const LaunchContext& c) {
      return tmc_pack_weights_f16(c.ptrs[0], c.ptrs[1], n, k, c.stream);
    };
    return true;
  }
  if (name == "gemm_packed") {
    // norm=1&eps: RMSNorm folded in (W packed with its gamma,
    // tmc_pack_weights_scaled_f16); residual=1: y = h(h(x W^T) + residual)
    // (inputs x, W, residual in y's layout).
    const int64_t b = param_int(p, "batch"), k = param_int(p, "in"), n = param_int(p, "out");
    const int od = param_dtype(p, "out_dtype", TMC_F16);
    const bool norm = param_int(p, "norm", 0) != 0, res = param_int(p, "residual", 0) != 0;
    const float eps = (float)param_double(p, "eps", 1e-6);
    NEED(b > 0 && k > 0 && n > 0 && (od == TMC_F16 || od == TMC_F32) && dt == TMC_F16,
         "gemm_packed needs batch, in, out > 0, dtype=f16 and out_dtype f16|f32.");
    NEED(!(norm && res) && (!res || od == TMC_F16),
         "gemm_packed: norm and residual exclude each other; a residual output is fp16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    int layout = 0;
    NEED(layout_param(p, layout), "packed GEMM key: x_layout / y_layout must be row_major or packed.");
    NEED(!(layout & TMC_LAYOUT_Y_PACKED) || od == TMC_F16, "gemm_packed: a packed output is fp16.");
    const size_t xc =
        (size_t)((layout & TMC_LAYOUT_X_PACKED) ? tmc_packed_activation_elements(b, k) : b * k);
    const size_t yc =
        (size_t)((layout & TMC_LAYOUT_Y_PACKED) ? tmc_packed_activation_elements(b, n) : b * n);
    const size_t wc = (size_t)tmc_packed_weight_elements(n, k);
    if (res) {
      s.inputs = {TMC_F16, TMC_F16, TMC_F16};
      s.counts = {xc, wc, yc, yc};
    } else {
      s.inputs = {TMC_F16, TMC_F16};
      s.counts = {xc, wc, yc};
    }
    s.outputs = {od};
    s.groups = (size_t)((n + 15) / 16);
    s.launch = [=](const LaunchContext& c) {
      if (norm)
        return tmc_gemm_packed_norm_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], od, b, k, n, eps, layout,
                                        &cfg, c.stream);
      if (res)
        return tmc_gemm_packed_residual_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], b, k, n,
                                            layout, &cfg, c.stream);
      return tmc_gemm_packed_ex_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], od, b, k, n, layout, &cfg,
                                    c.stream);
    };
    return true;
  }
  if (name == "pack_activations") {
    const int64_t r = param_int(p, "rows"), k = param_int(p, "cols");
    NEED(r > 0 && k > 0 && k % 8 == 0 && dt == TMC_F16,
         "pack_activations needs rows, cols (a multiple of 8) and f16.");
    s.inputs = {TMC_F16};
    s.outputs = {TMC_F16};
    s.counts = {(size_t)(r * k), (size_t)tmc_packed_activation_elements(r, k)};
    s.launch = [=](const LaunchContext& c) {
      return tmc_pack_activations_f16(c.ptrs[0], c.ptrs[1], r, k, 0, c.stream);
    };
    return true;
  }
  if (name == "qkv_rope_append_packed") {
    // Batched q.k.v projection over packed weights with RoPE + paged append
    // in its epilogue: inputs x, packed fused weight, cos, sin,
    // valid_lengths, block_tables, active; outputs q, key pool, value pool.
    const int64_t b = param_int(p, "batch"), h = param_int(p, "hidden"),
                  qh = param_int(p, "q_heads"), kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity"),
                  ps = param_int(p, "page_size");
    NEED(b > 0 && h > 0 && qh > 0 && kvh > 0 && d > 0 && cap > 0 && ps > 0 && dt == TMC_F16,
         "qkv_rope_append_packed needs batch, hidden, q_heads, head_dim, capacity, page_size "
         "and f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    int layout = 0;
    NEED(layout_param(p, layout) && !(layout & TMC_LAYOUT_Y_PACKED),
         "qkv_rope_append_packed: x_layout must be row_major or packed, no y_layout.");
    const int64_t mp = (cap + ps - 1) / ps, n = (qh + 2 * kvh) * d;
    // norm=1&eps: RMSNorm folded in (W packed with its gamma,
    // tmc_pack_weights_scaled_f16)
    const bool norm = param_int(p, "norm", 0) != 0;
    const float eps = (float)param_double(p, "eps", 1e-6);
    s.inputs = {TMC_F16, TMC_F16, TMC_F32, TMC_F32, TMC_I32, TMC_I32, TMC_I32};
    s.outputs = {TMC_F16, TMC_F16, TMC_F16};
    s.counts = {(size_t)((layout & TMC_LAYOUT_X_PACKED) ? tmc_packed_activation_elements(b, h) : b * h),
                (size_t)tmc_packed_weight_elements(n, h), (size_t)(cap * (d / 2)),
                (size_t)(cap * (d / 2)), (size_t)b, (size_t)(b * mp), 1, (size_t)(b * qh * d), 0, 0};
    s.launch = [=](const LaunchContext& c) {
      if (norm)
        return tmc_rmsnorm_qkv_rope_append_packed_f16(
            c.ptrs[0], c.ptrs[1], static_cast<const float*>(c.ptrs[2]),
            static_cast<const float*>(c.ptrs[3]), static_cast<const int32_t*>(c.ptrs[4]),
            static_cast<const int32_t*>(c.ptrs[5]), static_cast<const int32_t*>(c.ptrs[6]),
            c.ptrs[7], c.ptrs[8], c.ptrs[9], b, h, qh, kvh, d, cap, ps, mp, eps, layout, &cfg,
            c.stream);
      return tmc_qkv_rope_append_packed_f16(
          c.ptrs[0], c.ptrs[1], static_cast<const float*>(c.ptrs[2]),
          static_cast<const float*>(c.ptrs[3]), static_cast<const int32_t*>(c.ptrs[4]),
          static_cast<const int32_t*>(c.ptrs[5]), static_cast<const int32_t*>(c.ptrs[6]), c.ptrs[7],
          c.ptrs[8], c.ptrs[9], b, h, qh, kvh, d, cap, ps, mp, layout, &cfg, c.stream);
    };
    return true;
  }
  if (name == "gate_up_silu_packed") {
    const int64_t b = param_int(p, "batch"), h = param_int(p, "hidden"), f = param_int(p, "inter");
    NEED(b > 0 && h > 0 && f > 0 && dt == TMC_F16,
         "gate_up_silu_packed needs batch, hidden, inter and f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    int layout = 0;
    NEED(layout_param(p, layout), "packed GEMM key: x_layout / y_layout must be row_major or packed.");
    const size_t pe = (size_t)tmc_packed_weight_elements(f, h);
    // norm=1&eps: RMSNorm folded in (gate and up packed with its gamma,
    // tmc_pack_weights_scaled_f16)
    const bool norm = param_int(p, "norm", 0) != 0;
    const float eps = (float)param_double(p, "eps", 1e-6);
    s.inputs = {TMC_F16, TMC_F16, TMC_F16};
    s.outputs = {TMC_F16};
    s.groups = (size_t)((f + 15) / 16);
    s.counts = {(size_t)((layout & TMC_LAYOUT_X_PACKED) ? tmc_packed_activation_elements(b, h) : b * h),
                pe, pe,
                (size_t)((layout & TMC_LAYOUT_Y_PACKED) ? tmc_packed_activation_elements(b, f) : b * f)};
    s.launch = [=](const LaunchContext& c) {
      if (norm)
        return tmc_gate_up_silu_packed_norm_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], b, h,
                                                f, eps, layout, &cfg, c.stream);
      return tmc_gate_up_silu_packed_ex_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], b, h, f,
                                            layout, &cfg, c.stream);
    };
    return true;
  }
  if (name == "gate_up_silu") {
    const int64_t b = param_int(p, "batch"), h = param_int(p, "hidden"), f = param_int(p, "inter");
    NEED(b > 0 && h > 0 && f > 0 && dt == TMC_F16, "gate_up_silu needs batch, hidden, inter and f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    s.inputs = {TMC_F16, TMC_F16, TMC_F16};
    s.outputs = {TMC_F16};
    s.groups = (size_t)((f + 3) / 4);
    s.counts = {(size_t)(b * h), (size_t)(f * h), (size_t)(f * h), (size_t)(b * f)};
    s.launch = [=](const LaunchContext& c) {
      return tmc_gate_up_silu_f16_config(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], b, h, f,
                                         &cfg, c.stream);
    };
    return true;
  }
  if (name == "rmsnorm" || name == "add_rmsnorm") {
    const int64_t rows = param_int(p, "rows"), width = param_int(p, "width");
    const float eps = (float)param_double(p, "eps", 1e-5);
    NEED(rows > 0 && width > 0 && (dt == TMC_F16 || dt == TMC_F32), "rmsnorm needs rows, width, f16|f32.");
    // Tuner candidates: threads (64..1024, default 256) and variant
    // (default | two_pass, the fixed baseline at 256 threads).
    const int threads = (int)param_int(p, "threads", 256);
    const auto vit = p.find("variant");
    const std::string vname = vit == p.end() ? "default" : vit->second;
    NEED(threads == 64 || threads == 128 || threads == 256 || threads == 512 || threads == 1024,
         "rmsnorm threads must be 64, 128, 256, 512 or 1024.");
    NEED(vname == "default" || vname == "two_pass", "rmsnorm variant must be default or two_pass.");
    const int variant = vname == "two_pass" ? 1 : 0;
    const auto lit = p.find("out_layout");
    const bool packed_out = lit != p.end() && lit->second == "packed";
    NEED(lit == p.end() || lit->second == "packed" || lit->second == "row_major",
         "rmsnorm out_layout must be row_major or packed.");
    NEED(!packed_out || (dt == TMC_F16 && threads == 256 && variant == 0),
         "rmsnorm packed output needs f16 and the default 256-thread kernel.");
    s.groups = (size_t)rows;
    s.threads = (size_t)threads;
    if (packed_out) {
      const bool add = name == "add_rmsnorm";
      const size_t n_count = (size_t)tmc_packed_activation_elements(rows, width);
      s.inputs = add ? std::vector<int>{dt, dt, dt} : std::vector<int>{dt, dt};
      s.outputs = add ? std::vector<int>{dt, dt} : std::vector<int>{dt};
      s.counts = add ? std::vector<size_t>{(size_t)(rows * width), (size_t)(rows * width),
                                           (size_t)width, (size_t)(rows * width), n_count}
                     : std::vector<size_t>{(size_t)(rows * width), (size_t)width, n_count};
      s.launch = [=](const LaunchContext& c) {
        if (add)
          return tmc_add_rmsnorm_ex(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], c.ptrs[4], dt, rows,
                                    width, eps, TMC_LAYOUT_Y_PACKED, c.stream);
        return tmc_add_rmsnorm_ex(c.ptrs[0], nullptr, c.ptrs[1], nullptr, c.ptrs[2], dt, rows,
                                  width, eps, TMC_LAYOUT_Y_PACKED, c.stream);
      };
      return true;
    }
    if (name == "rmsnorm") {
      s.inputs = {dt, dt};
      s.outputs = {dt};
      s.counts = {(size_t)(rows * width), (size_t)width, (size_t)(rows * width)};
      s.launch = [=](const LaunchContext& c) {
        return tmc_rmsnorm_threads(c.ptrs[0], c.ptrs[1], c.ptrs[2], dt, rows, width, eps, threads,
                                   variant, c.stream);
      };
    } else {
      s.inputs = {dt, dt, dt};
      s.outputs = {dt, dt};
      s.counts = {(size_t)(rows * width), (size_t)(rows * width), (size_t)width,
                  (size_t)(rows * width), (size_t)(rows * width)};
      s.launch = [=](const LaunchContext& c) {
        return tmc_add_rmsnorm_threads(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], c.ptrs[4], dt,
                                       rows, width, eps, threads, variant, c.stream);
      };
    }
    return true;
  }
  if (name == "silu_mul" || name == "add" || name == "mul" || name == "silu") {
    // Element-wise ops of the decoder and of the graph path.  Without a
    // `threads` parameter add and silu_mul keep the decoder's launches;
    // with one (64, 128 or 256, the graph tuner's candidates) or for mul
    // and silu they run tmc_elementwise.
    const int64_t n = param_int(p, "count");
    NEED(n > 0 && (dt == TMC_F16 || dt == TMC_F32), "elementwise kernel needs count and f16|f32.");
    const bool explicit_threads = p.find("threads") != p.end();
    const int threads = (int)param_int(p, "threads", 256);
    NEED(threads == 64 || threads == 128 || threads == 256,
         "elementwise threads must be 64, 128 or 256.");
    const bool unary = name == "silu";
    s.inputs = unary ? std::vector<int>{dt} : std::vector<int>{dt, dt};
    s.outputs = {dt};
    s.threads = (size_t)threads;
    s.groups = (size_t)((n + threads - 1) / threads);
    s.counts = unary ? std::vector<size_t>{(size_t)n, (size_t)n}
                     : std::vector<size_t>{(size_t)n, (size_t)n, (size_t)n};
    const int op = name == "add" ? 0 : name == "mul" ? 1 : name == "silu" ? 2 : 3;
    if (!explicit_threads && (op == 0 || op == 3)) {
      s.launch = [=](const LaunchContext& c) {
        return op == 3 ? tmc_silu_mul(c.ptrs[0], c.ptrs[1], c.ptrs[2], dt, n, c.stream)
                       : tmc_add(c.ptrs[0], c.ptrs[1], c.ptrs[2], dt, n, c.stream);
      };
    } else {
      s.launch = [=](const LaunchContext& c) {
        return unary ? tmc_elementwise(op, c.ptrs[0], nullptr, c.ptrs[1], dt, n, threads, c.stream)
                     : tmc_elementwise(op, c.ptrs[0], c.ptrs[1], c.ptrs[2], dt, n, threads,
                                       c.stream);
      };
    }
    return true;
  }
  if (name == "embedding") {
    const int64_t rows = param_int(p, "rows"), h = param_int(p, "hidden"), v = param_int(p, "vocab");
    NEED(rows > 0 && h > 0 && v > 0, "embedding needs rows, hidden, vocab.");
    s.inputs = {TMC_I32, dt};
    s.outputs = {dt};
    s.groups = (size_t)rows;
    s.counts = {(size_t)rows, (size_t)(v * h), (size_t)(rows * h)};
    s.launch = [=](const LaunchContext& c) {
      return tmc_embedding(static_cast<const int32_t*>(c.ptrs[0]), c.ptrs[1], c.ptrs[2], dt, rows,
                           h, v, c.stream);
    };
    return true;
  }
  if (name == "rope") {
    const int64_t b = param_int(p, "batch"), sq = param_int(p, "seq"), hd = param_int(p, "heads"),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity");
    NEED(b > 0 && sq > 0 && hd > 0 && d > 0 && cap > 0, "rope needs batch, seq, heads, head_dim, capacity.");
    s.inputs = {dt, TMC_F32, TMC_F32, TMC_I32};
    s.outputs = {dt};
    s.counts = {(size_t)(b * sq * hd * d), (size_t)(cap * (d / 2)), (size_t)(cap * (d / 2)), 1,
                (size_t)(b * sq * hd * d)};
    s.launch = [=](const LaunchContext& c) {
      return tmc_rope(c.ptrs[0], static_cast<const float*>(c.ptrs[1]),
                      static_cast<const float*>(c.ptrs[2]), static_cast<const int32_t*>(c.ptrs[3]),
                      c.ptrs[4], dt, b, sq, hd, d, cap, c.stream);
    };
    return true;
  }
  if (name == "serving_rope") {
    const int64_t b = param_int(p, "max_batch"), hd = param_int(p, "heads"),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity");
    NEED(b > 0 && hd > 0 && d > 0 && cap > 0, "serving_rope needs max_batch, heads, head_dim, capacity.");
    s.inputs = {dt, TMC_F32, TMC_F32, TMC_I32, TMC_I32};
    s.outputs = {dt};
    s.counts = {(size_t)(b * hd * d), (size_t)(cap * (d / 2)), (size_t)(cap * (d / 2)), (size_t)b, 1,
                (size_t)(b * hd * d)};
    s.launch = [=](const LaunchContext& c) {
      return tmc_serving_rope(c.ptrs[0], static_cast<const float*>(c.ptrs[1]),
                              static_cast<const float*>(c.ptrs[2]),
                              static_cast<const int32_t*>(c.ptrs[3]),
                              static_cast<const int32_t*>(c.ptrs[4]), c.ptrs[5], dt, b, hd, d, cap,
                              c.stream);
    };
    return true;
  }
  if (name == "kv_append" || name == "paged_kv_append") {
    const int64_t b = param_int(p, "batch"), sq = param_int(p, "seq"), hd = param_int(p, "heads"),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity");
    const int hm = (int)param_int(p, "head_major", 0);
    NEED(b > 0 && sq > 0 && hd > 0 && d > 0 && cap > 0, "kv_append needs batch, seq, heads, head_dim, capacity.");
    if (name == "kv_append") {
      s.inputs = {dt, TMC_I32};
      s.outputs = {dt};
      s.counts = {(size_t)(b * sq * hd * d), 1, (size_t)(b * hd * cap * d)};
      s.launch = [=](const LaunchContext& c) {
        return tmc_kv_append(c.ptrs[0], static_cast<const int32_t*>(c.ptrs[1]), c.ptrs[2], dt, b,
                             sq, hd, d, cap, hm, c.stream);
      };
    } else {
      const int64_t ps = param_int(p, "page_size");
      NEED(ps > 0, "paged_kv_append needs page_size.");
      s.inputs = {dt, TMC_I32, TMC_I32};
      s.outputs = {dt};
      s.counts = {(size_t)(b * sq * hd * d), 1, (size_t)((cap + ps - 1) / ps), 0};
      s.launch = [=](const LaunchContext& c) {
        return tmc_paged_kv_append(c.ptrs[0], static_cast<const int32_t*>(c.ptrs[1]),
                                   static_cast<const int32_t*>(c.ptrs[2]), c.ptrs[3], dt, b, sq,
                                   hd, d, cap, ps, hm, c.stream);
      };
    }
    return true;
  }
  if (name == "serving_kv_append") {
    const int64_t b = param_int(p, "max_batch"), hd = param_int(p, "heads"),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity"),
                  ps = param_int(p, "page_size");
    const int hm = (int)param_int(p, "head_major", 0);
    NEED(b > 0 && hd > 0 && d > 0 && cap > 0 && ps > 0, "serving_kv_append needs max_batch, heads, head_dim, capacity, page_size.");
    s.inputs = {dt, TMC_I32, TMC_I32, TMC_I32};
    s.outputs = {dt};
    s.counts = {(size_t)(b * hd * d), (size_t)b, (size_t)(b * ((cap + ps - 1) / ps)), 1, 0};
    s.launch = [=](const LaunchContext& c) {
      return tmc_serving_kv_append(c.ptrs[0], static_cast<const int32_t*>(c.ptrs[1]),
                                   static_cast<const int32_t*>(c.ptrs[2]),
                                   static_cast<const int32_t*>(c.ptrs[3]), c.ptrs[4], dt, b, hd,
                                   d, cap, ps, hm, c.stream);
    };
    return true;
  }
  if (name == "decode_rope_append") {
    const int64_t b = param_int(p, "max_batch"), qh = param_int(p, "q_heads"),
                  kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity"),
                  ps = param_int(p, "page_size");
    NEED(b > 0 && qh > 0 && kvh > 0 && d > 0 && cap > 0 && ps > 0,
         "decode_rope_append needs max_batch, q_heads, head_dim, capacity, page_size.");
    const int64_t mp = (cap + ps - 1) / ps;
    // inputs: qkv, cos, sin, valid_lengths, block_tables, active; outputs: q, key pool, value pool
    s.inputs = {dt, TMC_F32, TMC_F32, TMC_I32, TMC_I32, TMC_I32};
    s.outputs = {dt, dt, dt};
    s.counts = {(size_t)(b * (qh + 2 * kvh) * d), (size_t)(cap * (d / 2)),
                (size_t)(cap * (d / 2)), (size_t)b, (size_t)(b * mp), 1, (size_t)(b * qh * d), 0, 0};
    s.launch = [=](const LaunchContext& c) {
      return tmc_decode_rope_append(c.ptrs[0], static_cast<const float*>(c.ptrs[1]),
                                    static_cast<const float*>(c.ptrs[2]),
                                    static_cast<const int32_t*>(c.ptrs[3]),
                                    static_cast<const int32_t*>(c.ptrs[4]),
                                    static_cast<const int32_t*>(c.ptrs[5]), c.ptrs[6], c.ptrs[7],
                                    c.ptrs[8], dt, b, qh, kvh, d, cap, ps, mp, c.stream);
    };
    return true;
  }
  if (name == "add_rmsnorm_qkv_rope_append" || name == "rmsnorm_qkv_rope_append") {
    // Batch-1 norm + q.k.v projection + RoPE + paged append: inputs
    // residual[, update], gamma, fused weight, cos, sin, valid_lengths,
    // block_table, active; outputs [sum,] q, key pool, value pool.
    const bool add = name.rfind("add_", 0) == 0;
    const int64_t h = param_int(p, "hidden"), qh = param_int(p, "q_heads"),
                  kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity"),
                  ps = param_int(p, "page_size");
    const float eps = (float)param_double(p, "eps", 1e-5);
    NEED(h > 0 && qh > 0 && kvh > 0 && d > 0 && cap > 0 && ps > 0 && dt == TMC_F16,
         "rmsnorm_qkv_rope_append needs hidden, q_heads, head_dim, capacity, page_size and "
         "dtype=f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    const int64_t mp = (cap + ps - 1) / ps;
    s.inputs = add ? std::vector<int>{TMC_F16, TMC_F16} : std::vector<int>{TMC_F16};
    s.inputs.insert(s.inputs.end(), {TMC_F16, TMC_F16, TMC_F32, TMC_F32, TMC_I32, TMC_I32, TMC_I32});
    s.outputs = add ? std::vector<int>{TMC_F16, TMC_F16, TMC_F16, TMC_F16}
                    : std::vector<int>{TMC_F16, TMC_F16, TMC_F16};
    s.counts = add ? std::vector<size_t>{(size_t)h, (size_t)h} : std::vector<size_t>{(size_t)h};
    s.counts.insert(s.counts.end(), {(size_t)h, (size_t)((qh + 2 * kvh) * d * h),
                                     (size_t)(cap * (d / 2)), (size_t)(cap * (d / 2)), 1,
                                     (size_t)mp, 1});
    if (add) s.counts.push_back((size_t)h);
    s.counts.insert(s.counts.end(), {(size_t)(qh * d), 0, 0});
    s.launch = [=](const LaunchContext& c) {
      const int o = add ? 1 : 0;  // index shift past the update input
      return tmc_add_rmsnorm_qkv_rope_append_f16(
          c.ptrs[0], add ? c.ptrs[1] : nullptr, c.ptrs[1 + o], c.ptrs[2 + o],
          add ? c.ptrs[9] : nullptr, static_cast<const float*>(c.ptrs[3 + o]),
          static_cast<const float*>(c.ptrs[4 + o]), static_cast<const int32_t*>(c.ptrs[5 + o]),
          static_cast<const int32_t*>(c.ptrs[6 + o]), static_cast<const int32_t*>(c.ptrs[7 + o]),
          c.ptrs[8 + 2 * o], c.ptrs[9 + 2 * o], c.ptrs[10 + 2 * o], h, qh, kvh, d, cap, ps, eps,
          &cfg, c.stream);
    };
    return true;
  }
  if (name == "qkv_rope_append") {
    // Batch-1 q.k.v projection with RoPE and the paged K/V append fused in
    // its epilogue: inputs x, fused weight, cos, sin, valid_lengths,
    // block_table, active; outputs q, key pool, value pool.
    const int64_t h = param_int(p, "hidden"), qh = param_int(p, "q_heads"),
                  kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity"),
                  ps = param_int(p, "page_size");
    NEED(h > 0 && qh > 0 && kvh > 0 && d > 0 && cap > 0 && ps > 0 && dt == TMC_F16,
         "qkv_rope_append needs hidden, q_heads, head_dim, capacity, page_size and dtype=f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    const int64_t mp = (cap + ps - 1) / ps;
    s.inputs = {TMC_F16, TMC_F16, TMC_F32, TMC_F32, TMC_I32, TMC_I32, TMC_I32};
    s.outputs = {TMC_F16, TMC_F16, TMC_F16};
    s.counts = {(size_t)h, (size_t)((qh + 2 * kvh) * d * h), (size_t)(cap * (d / 2)),
                (size_t)(cap * (d / 2)), 1, (size_t)mp, 1, (size_t)(qh * d), 0, 0};
    s.launch = [=](const LaunchContext& c) {
      return tmc_qkv_rope_append_f16(c.ptrs[0], c.ptrs[1], static_cast<const float*>(c.ptrs[2]),
                                     static_cast<const float*>(c.ptrs[3]),
                                     static_cast<const int32_t*>(c.ptrs[4]),
                                     static_cast<const int32_t*>(c.ptrs[5]),
                                     static_cast<const int32_t*>(c.ptrs[6]), c.ptrs[7], c.ptrs[8],
                                     c.ptrs[9], h, qh, kvh, d, cap, ps, &cfg, c.stream);
    };
    return true;
  }
  if (name == "decode_attention") {
    const int64_t b = param_int(p, "batch"), qh = param_int(p, "q_heads"),
                  kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity");
    NEED(b > 0 && qh > 0 && kvh > 0 && d > 0 && cap > 0, "decode_attention needs batch, q_heads, head_dim, capacity.");
    s.inputs = {dt, dt, dt, TMC_I32};
    s.outputs = {dt};
    s.counts = {(size_t)(b * qh * d), (size_t)(b * kvh * cap * d), (size_t)(b * kvh * cap * d), 1,
                (size_t)(b * qh * d)};
    s.workspace_bytes = tmc_attention_workspace_bytes(b, qh, kvh, d, cap);
    s.launch = [=](const LaunchContext& c) {
      return tmc_decode_attention(c.ptrs[0], c.ptrs[1], c.ptrs[2],
                                  static_cast<const int32_t*>(c.ptrs[3]), c.ptrs[4], dt, b, qh, kvh,
                                  d, cap, c.workspace, c.workspace_bytes, c.stream);
    };
    return true;
  }
  if (name == "paged_attention") {
    const int64_t b = param_int(p, "max_batch"), qh = param_int(p, "q_heads"),
                  kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), ps = param_int(p, "page_size"),
                  mp = param_int(p, "max_pages");
    NEED(b > 0 && qh > 0 && kvh > 0 && d > 0 && ps > 0 && mp > 0,
         "paged_attention needs max_batch, q_heads, head_dim, page_size, max_pages.");
    const int64_t head_stride = param_int(p, "head_stride", ps * d);
    const int64_t page_stride = param_int(p, "page_stride", kvh * ps * d);
    const auto lit = p.find("out_layout");
    const bool packed_out = lit != p.end() && lit->second == "packed";
    NEED(lit == p.end() || packed_out || lit->second == "row_major",
         "paged_attention out_layout must be row_major or packed.");
    NEED(!packed_out || dt == TMC_F16, "paged_attention packed output needs f16.");
    const int layout = packed_out ? TMC_LAYOUT_Y_PACKED : 0;
    s.inputs = {dt, dt, dt, TMC_I32, TMC_I32, TMC_I32};
    s.outputs = {dt};
    s.counts = {(size_t)(b * qh * d), 0, 0, (size_t)b, (size_t)(b * mp), 1,
                packed_out ? (size_t)tmc_packed_activation_elements(b, qh * d)
                           : (size_t)(b * qh * d)};
    s.workspace_bytes = tmc_attention_workspace_bytes(b, qh, kvh, d, ps * mp);
    s.launch = [=](const LaunchContext& c) {
      const int64_t pool_pages =
          (int64_t)(std::min(c.counts[1], c.counts[2]) / (size_t)page_stride);
      return tmc_paged_decode_attention_ex(
          c.ptrs[0], c.ptrs[1], c.ptrs[2], static_cast<const int32_t*>(c.ptrs[3]),
          static_cast<const int32_t*>(c.ptrs[4]), static_cast<const int32_t*>(c.ptrs[5]),
          c.ptrs[6], dt, b, qh, kvh, d, ps, mp, pool_pages, page_stride, head_stride,
          c.workspace, c.workspace_bytes, layout, c.stream);
    };
    return true;
  }
  if (name == "paged_attention_output") {
    // Batch-1 paged attention + output projection (+ residual when
    // residual=1): inputs q, key pool, value pool, lengths, block table,
    // active count, W [out, q_heads*head_dim] (, residual [out]); output y.
    const int64_t qh = param_int(p, "q_heads"), kvh = param_int(p, "kv_heads", qh),
                  d = param_int(p, "head_dim"), ps = param_int(p, "page_size"),
                  mp = param_int(p, "max_pages"), n = param_int(p, "out");
    const bool res = param_int(p, "residual", 0) != 0;
    NEED(qh > 0 && kvh > 0 && d > 0 && ps > 0 && mp > 0 && n > 0 && dt == TMC_F16,
         "paged_attention_output needs q_heads, head_dim, page_size, max_pages, out and "
         "dtype=f16.");
    const int64_t head_stride = param_int(p, "head_stride", ps * d);
    const int64_t page_stride = param_int(p, "page_stride", kvh * ps * d);
    s.inputs = {dt, dt, dt, TMC_I32, TMC_I32, TMC_I32, dt};
    s.counts = {(size_t)(qh * d), 0, 0, 1, (size_t)mp, 1, (size_t)(n * qh * d)};
    if (res) {
      s.inputs.push_back(dt);
      s.counts.push_back((size_t)n);
    }
    s.outputs = {dt};
    s.counts.push_back((size_t)n);
    s.workspace_bytes = tmc_attention_output_workspace_bytes(qh, kvh, n);
    NEED(s.workspace_bytes > 0,
         "paged_attention_output: unsupported head grouping or output width.");
    s.launch = [=](const LaunchContext& c) {
      const int64_t pool_pages =
          (int64_t)(std::min(c.counts[1], c.counts[2]) / (size_t)page_stride);
      return tmc_paged_attention_output_f16(
          c.ptrs[0], c.ptrs[1], c.ptrs[2], static_cast<const int32_t*>(c.ptrs[3]),
          static_cast<const int32_t*>(c.ptrs[4]), static_cast<const int32_t*>(c.ptrs[5]),
          c.ptrs[6], res ? c.ptrs[7] : nullptr, c.ptrs[res ? 8 : 7], qh, kvh, d, ps, mp,
          pool_pages, page_stride, head_stride, n, c.workspace, c.workspace_bytes, c.stream);
    };
    return true;
  }
  if (name == "gemm_rows") {
    // Prompt GEMM y[m, out] = x[m, in] w[out, in]^T; workspace=1 binds a
    // trailing int32 scratch input of tmc_gemm_rows_workspace_bytes().
    const int64_t m = param_int(p, "m"), k = param_int(p, "in"), n = param_int(p, "out");
    const int od = param_dtype(p, "out_dtype", TMC_F16);
    const bool ws = param_int(p, "workspace", 0) != 0;
    NEED(m > 0 && k > 0 && n > 0 && dt == TMC_F16 && (od == TMC_F16 || od == TMC_F32),
         "gemm_rows needs m, in, out > 0, dtype=f16 and out_dtype f16|f32.");
    const size_t ws_bytes = ws ? tmc_gemm_rows_workspace_bytes() : 0;
    s.inputs = {TMC_F16, TMC_F16};
    s.counts = {(size_t)(m * k), (size_t)(n * k)};
    if (ws) {
      s.inputs.push_back(TMC_I32);
      s.counts.push_back(ws_bytes / 4);
    }
    s.outputs = {od};
    s.counts.push_back((size_t)(m * n));
    s.groups = (size_t)(((m + 127) / 128) * ((n + 127) / 128));
    s.launch = [=](const LaunchContext& c) {
      return tmc_gemm_rows_f16(c.ptrs[0], c.ptrs[1], c.ptrs[ws ? 3 : 2], od, m, k, n,
                               ws ? c.ptrs[2] : nullptr, ws_bytes, c.stream);
    };
    return true;
  }
  if (name == "prefill_rope_append") {
    const int64_t rows = param_int(p, "rows"), qh = param_int(p, "q_heads"),
                  kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), cap = param_int(p, "capacity"),
                  ps = param_int(p, "page_size");
    NEED(rows > 0 && qh > 0 && kvh > 0 && d > 0 && cap > 0 && ps > 0,
         "prefill_rope_append needs rows, q_heads, head_dim, capacity, page_size.");
    const int64_t mp = (cap + ps - 1) / ps;
    // tables=N > 0: N table rows and a row table (int32 [rows]) after them.
    const int64_t tr = param_int(p, "tables", 0);
    NEED(tr >= 0 && tr < (1 << 20), "prefill_rope_append: tables must be >= 0.");
    // inputs: qkv, cos, sin, valid_lengths, block table(s)[, row table], active;
    // outputs: q, key pool, value pool
    s.inputs = {dt, TMC_F32, TMC_F32, TMC_I32, TMC_I32};
    s.counts = {(size_t)(rows * (qh + 2 * kvh) * d), (size_t)(cap * (d / 2)),
                (size_t)(cap * (d / 2)), (size_t)rows, (size_t)(mp * (tr ? tr : 1))};
    if (tr) {
      s.inputs.push_back(TMC_I32);
      s.counts.push_back((size_t)rows);
    }
    s.inputs.push_back(TMC_I32);
    s.counts.push_back(1);
    s.outputs = {dt, dt, dt};
    s.counts.insert(s.counts.end(), {(size_t)(rows * qh * d), 0, 0});
    const int a = tr ? 6 : 5;  // index of the active count
    s.launch = [=](const LaunchContext& c) {
      const auto i32 = [&](int i) { return static_cast<const int32_t*>(c.ptrs[i]); };
      if (tr)
        return tmc_prefill_rope_append_rows(c.ptrs[0], static_cast<const float*>(c.ptrs[1]),
                                            static_cast<const float*>(c.ptrs[2]), i32(3), i32(4),
                                            i32(5), tr, i32(a), c.ptrs[a + 1], c.ptrs[a + 2],
                                            c.ptrs[a + 3], dt, rows, qh, kvh, d, cap, ps, mp,
                                            c.stream);
      return tmc_prefill_rope_append(c.ptrs[0], static_cast<const float*>(c.ptrs[1]),
                                     static_cast<const float*>(c.ptrs[2]), i32(3), i32(4), i32(a),
                                     c.ptrs[a + 1], c.ptrs[a + 2], c.ptrs[a + 3], dt, rows, qh, kvh,
                                     d, cap, ps, mp, c.stream);
    };
    return true;
  }
  if (name == "prefill_attention") {
    const int64_t rows = param_int(p, "rows"), qh = param_int(p, "q_heads"),
                  kvh = param_int(p, "kv_heads", param_int(p, "q_heads")),
                  d = param_int(p, "head_dim"), ps = param_int(p, "page_size"),
                  mp = param_int(p, "max_pages");
    NEED(rows > 0 && qh > 0 && kvh > 0 && d > 0 && ps > 0 && mp > 0 && dt == TMC_F16,
         "prefill_attention needs rows, q_heads, head_dim, page_size, max_pages and dtype=f16.");
    const int64_t head_stride = param_int(p, "head_stride", ps * d);
    const int64_t page_stride = param_int(p, "page_stride", kvh * ps * d);
    const int64_t tr = param_int(p, "tables", 0);  // > 0: table rows + a row table
    NEED(tr >= 0 && tr < (1 << 20), "prefill_attention: tables must be >= 0.");
    // inputs: q, key pool, value pool, valid_lengths, block table(s)[, row table], active;
    // output: context
    s.inputs = {dt, dt, dt, TMC_I32, TMC_I32};
    s.counts = {(size_t)(rows * qh * d), 0, 0, (size_t)rows, (size_t)(mp * (tr ? tr : 1))};
    if (tr) {
      s.inputs.push_back(TMC_I32);
      s.counts.push_back((size_t)rows);
    }
    s.inputs.push_back(TMC_I32);
    s.counts.push_back(1);
    s.outputs = {dt};
    s.counts.push_back((size_t)(rows * qh * d));
    const int a = tr ? 6 : 5;  // index of the active count
    s.launch = [=](const LaunchContext& c) {
      const int64_t pool_pages =
          (int64_t)(std::min(c.counts[1], c.counts[2]) / (size_t)page_stride);
      const auto i32 = [&](int i) { return static_cast<const int32_t*>(c.ptrs[i]); };
      return tmc_prefill_attention_rows_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], i32(3), i32(4),
                                            tr ? i32(5) : nullptr, tr ? tr : 1, i32(a),
                                            c.ptrs[a + 1], rows, qh, kvh, d, ps, mp, pool_pages,
                                            page_stride, head_stride, c.stream);
    };
    return true;
  }
  if (name == "argmax") {
    const int64_t rows = param_int(p, "rows"), v = param_int(p, "vocab");
    NEED(rows > 0 && v > 0, "argmax needs rows and vocab.");
    s.inputs = {TMC_F32};
    s.outputs = {TMC_I32};
    s.groups = (size_t)rows;
    s.counts = {(size_t)(rows * v), (size_t)rows};
    s.launch = [=](const LaunchContext& c) {
      return tmc_argmax_f32(static_cast<const float*>(c.ptrs[0]), static_cast<int32_t*>(c.ptrs[1]),
                            rows, v, c.stream);
    };
    return true;
  }
  if (name == "rmsnorm_lm_head_partial_argmax") {
    // Token-only LM head at batch 1 (emitLMHeadPartialArgmax): inputs the
    // stored residual row, the final norm's gamma and W; output the
    // partial-argmax workspace.
    const int64_t k = param_int(p, "in"), n = param_int(p, "out");
    const float eps = (float)param_double(p, "eps", 1e-6);
    NEED(param_int(p, "batch", 1) == 1 && k > 0 && n > 0 && dt == TMC_F16,
         "rmsnorm_lm_head_partial_argmax needs batch=1, in, out > 0 and f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    const size_t ws = tmc_lm_head_argmax_workspace_bytes(1, n);
    NEED(ws > 0, "rmsnorm_lm_head_partial_argmax: vocabulary out of range.");
    s.inputs = {TMC_F16, TMC_F16, TMC_F16};
    s.outputs = {TMC_F32};
    s.counts = {(size_t)k, (size_t)k, (size_t)(n * k), ws / 4};
    s.groups = (size_t)((n + 7) / 8);
    s.launch = [=](const LaunchContext& c) {
      return tmc_rmsnorm_lm_head_partial_argmax_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], c.ptrs[3], ws,
                                                    k, n, eps, &cfg, c.stream);
    };
    return true;
  }
  if (name == "lm_head_partial_argmax_packed") {
    // Token-only LM head above batch 1 on the gamma-scaled packed weights:
    // inputs x (x_layout) and W; output the partial-argmax workspace.
    const int64_t b = param_int(p, "batch"), k = param_int(p, "in"), n = param_int(p, "out");
    const float eps = (float)param_double(p, "eps", 1e-6);
    NEED(b > 0 && k > 0 && n > 0 && dt == TMC_F16,
         "lm_head_partial_argmax_packed needs batch, in, out > 0 and f16.");
    tmc_gemv_config cfg{};
    NEED(gemv_config_param(p, cfg), "GEMV key: algorithm must be 0..5.");
    int layout = 0;
    NEED(layout_param(p, layout) && !(layout & TMC_LAYOUT_Y_PACKED),
         "lm_head_partial_argmax_packed: x_layout must be row_major or packed (no y_layout).");
    const size_t ws = tmc_lm_head_argmax_workspace_bytes(b, n);
    NEED(ws > 0, "lm_head_partial_argmax_packed: batch or vocabulary out of range.");
    const size_t xc =
        (size_t)((layout & TMC_LAYOUT_X_PACKED) ? tmc_packed_activation_elements(b, k) : b * k);
    s.inputs = {TMC_F16, TMC_F16};
    s.outputs = {TMC_F32};
    s.counts = {xc, (size_t)tmc_packed_weight_elements(n, k), ws / 4};
    s.groups = (size_t)((n + 15) / 16);
    s.launch = [=](const LaunchContext& c) {
      return tmc_lm_head_partial_argmax_packed_norm_f16(c.ptrs[0], c.ptrs[1], c.ptrs[2], ws, b, k,
                                                        n, eps, layout, &cfg, c.stream);
    };
    return true;
  }
  if (name == "lm_head_final_argmax") {
    // emitLMHeadFinalArgmax: input the partial-argmax workspace, output the
    // rows' tokens.
    const int64_t rows = param_int(p, "rows"), v = param_int(p, "vocab");
    const size_t ws = tmc_lm_head_argmax_workspace_bytes(rows, v);
    NEED(rows > 0 && v > 0 && ws > 0, "lm_head_final_argmax needs rows and vocab.");
    s.inputs = {TMC_F32};
    s.outputs = {TMC_I32};
    s.groups = (size_t)rows;
    s.counts = {ws / 4, (size_t)rows};
    s.launch = [=](const LaunchContext& c) {
      return tmc_lm_head_final_argmax(c.ptrs[0], ws, static_cast<int32_t*>(c.ptrs[1]), rows, v,
                                      c.stream);
    };
    return true;
  }
  set_error("Unknown gfx950 kernel '" + name + "'.");
  return false;
}

#undef NEED

int consume_failure(tmc_runtime* rt) {
  if (rt->fail_next > 0) {
    --rt->fail_next;
    set_error("Injected execution failure (tmc_rt_fail_next).");
    return 1;
  }
  return 0;
}

}  // namespace

// ====================================================================== C ABI
extern "C" const char* tmc_last_error(void) { return g_error.c_str(); }

extern "C" int tmc_rt_create(tmc_runtime** out) {
  clear_error();
  if (!out) return fail("tmc_rt_create: null output.");
  auto rt = std::make_unique<tmc_runtime>();
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    rt->init_error = "No HIP device was found.";
  } else if (hipGetDeviceProperties(&rt->props, 0) != hipSuccess) {
    rt->init_error = "hipGetDeviceProperties failed.";
  } else if (std::string(rt->props.gcnArchName).rfind("gfx950", 0) != 0) {
    rt->init_error = std::string("Device ") + rt->props.gcnArchName +
                     " is not gfx950; this library holds gfx950 code only.";
  } else if (hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking) != hipSuccess) {
    rt->init_error = "hipStreamCreate failed.";
  } else {
    rt->available = true;
    rt->device_name = rt->props.name;
    if (rt->device_name.empty()) rt->device_name = rt->props.gcnArchName;
  }
  *out = rt.release();
  return 0;
}

extern "C" void tmc_rt_destroy(tmc_runtime* rt) {
  if (!rt) return;
  if (rt->stream) {
    (void)hipStreamSynchronize(rt->stream);
    (void)hipStreamDestroy(rt->stream);
  }
  if (rt->staged_done) (void)hipEventDestroy(rt->staged_done);
  if (rt->staging) (void)hipHostFree(rt->staging);
  delete rt;
}

extern "C" int tmc_rt_is_available(const tmc_runtime* rt) { return rt && rt->available; }
extern "C" const char* tmc_rt_device_name(const tmc_runtime* rt) {
  return rt ? rt->device_name.c_str() : "";
}
extern "C" const char* tmc_rt_init_error(const tmc_runtime* rt) {
  return rt ? rt->init_error.c_str() : "null runtime";
}
extern "C" void* tmc_rt_stream(const tmc_runtime* rt) { return rt ? (void*)rt->stream : nullptr; }
extern "C" int tmc_rt_synchronize(tmc_runtime* rt) {
  clear_error();
  if (!rt) return fail("tmc_rt_synchronize: null runtime.");
  if (!rt->available) return fail(rt->init_error);
  return hip_ok(hipStreamSynchronize(rt->stream), "stream synchronize");
}

extern "C" void tmc_rt_fail_next(tmc_runtime* rt, int count) {
  if (rt) rt->fail_next = count;
}

extern "C" int tmc_rt_device_info(const tmc_runtime* rt, tmc_hardware_info* info) {
  if (!rt || !info) return fail("tmc_rt_device_info: null argument.");
  if (!rt->available) return fail(rt->init_error);
  info->max_threads_per_threadgroup = (size_t)rt->props.maxThreadsPerBlock;
  info->max_threadgroup_memory_length = (size_t)rt->props.sharedMemPerBlock;
  info->max_buffer_length = (size_t)rt->props.totalGlobalMem;
  info->supports_bfloat16 = 1;
  info->compute_units = rt->props.multiProcessorCount;
  info->wave_size = rt->props.warpSize;
  return 0;
}

extern "C" int tmc_buf_create(tmc_runtime* rt, size_t count, int dtype, const float* init,
                              tmc_buffer** out) {
  clear_error();
  if (!rt || !out) return fail("tmc_buf_create: null argument.");
  if (!rt->available) return fail(rt->init_error);
  if (!valid_dtype(dtype)) return fail("tmc_buf_create: unknown dtype.");
  const size_t bytes = count * element_bytes(dtype);
  if (count == 0 || bytes / element_bytes(dtype) != count || bytes > rt->props.totalGlobalMem)
    return fail("Buffer size is zero or exceeds the device limit.");
  auto buf = std::make_unique<tmc_buffer>();
  buf->rt = rt;
  buf->count = count;
  buf->dtype = dtype;
  if (hip_ok(hipMalloc(&buf->ptr, bytes), "Failed to allocate a device buffer")) return 1;
  int rc;
  if (init) {
    const auto host = encode(init, count, dtype);
    rc = hip_ok(hipMemcpy(buf->ptr, host.data(), bytes, hipMemcpyHostToDevice), "buffer upload");
  } else {
    rc = fill_sentinel(buf->ptr, count, dtype, true, rt->stream);
    if (!rc) rc = hip_ok(hipStreamSynchronize(rt->stream), "buffer fill");
  }
  if (rc) {
    (void)hipFree(buf->ptr);
    return 1;
  }
  *out = buf.release();
  return 0;
}

extern "C" int tmc_buf_wrap(tmc_runtime* rt, void* device_ptr, size_t count, int dtype,
                            tmc_buffer** out) {
  clear_error();
  if (!rt || !out || !device_ptr || count == 0 || !valid_dtype(dtype))
    return fail("tmc_buf_wrap: invalid argument.");
  auto buf = std::make_unique<tmc_buffer>();
  buf->rt = rt;
  buf->ptr = device_ptr;
  buf->count = count;
  buf->dtype = dtype;
  buf->owned = false;
  *out = buf.release();
  return 0;
}

extern "C" int tmc_buf_write(tmc_buffer* buf, const float* data, size_t count, size_t offset) {
  clear_error();
  if (!buf) return fail("Buffer is missing or belongs to another device.");
  if (!data || count == 0 || offset > buf->count || count > buf->count - offset)
    return fail("Host update range is invalid for the device buffer.");
  const auto host = encode(data, count, buf->dtype);
  const size_t eb = element_bytes(buf->dtype);
  // Ordered after earlier work on the runtime stream, complete on return.
  if (hip_ok(hipMemcpyAsync(static_cast<char*>(buf->ptr) + offset * eb, host.data(), count * eb,
                            hipMemcpyHostToDevice, buf->rt->stream),
             "buffer write"))
    return 1;
  return hip_ok(hipStreamSynchronize(buf->rt->stream), "buffer write");
}

extern "C" int tmc_buf_write_raw(tmc_buffer* buf, const void* data, size_t count, size_t offset) {
  clear_error();
  if (!buf || !data || count == 0 || offset > buf->count || count > buf->count - offset)
    return fail("tmc_buf_write_raw: invalid range.");
  const size_t eb = element_bytes(buf->dtype);
  if (hip_ok(hipMemcpyAsync(static_cast<char*>(buf->ptr) + offset * eb, data, count * eb,
                            hipMemcpyHostToDevice, buf->rt->stream),
             "raw write"))
    return 1;
  return hip_ok(hipStreamSynchronize(buf->rt->stream), "raw write");
}

namespace {
constexpr size_t kStagingBytes = size_t(4) << 20;

bool stream_captured(const tmc_runtime* rt) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(rt->stream, &capture) == hipSuccess &&
         capture != hipStreamCaptureStatusNone;
}

// `bytes` (rounded up to 256) of the runtime's pinned staging area for work
// queued next on the runtime stream; the caller records staged_done after
// that work.  Waits only when the area is full and its last user has not run.
int stage_reserve(tmc_runtime* rt, size_t bytes, char*& slot_out) {
  const size_t slot = (bytes + 255) / 256 * 256;
  if (!rt->staging) {
    void* pinned = nullptr;
    if (hip_ok(hipHostMalloc(&pinned, kStagingBytes, hipHostMallocDefault), "staging allocation"))
      return 1;
    void* mapped = nullptr;
    if (hip_ok(hipHostGetDevicePointer(&mapped, pinned, 0), "staging device address") ||
        hip_ok(hipEventCreateWithFlags(&rt->staged_done, hipEventDisableTiming), "staging event")) {
      (void)hipHostFree(pinned);
      return 1;
    }
    rt->staging = static_cast<char*>(pinned);
    rt->staging_device = static_cast<char*>(mapped);
    rt->staged = 0;
  }
  if (rt->staged != 0) {
    const hipError_t state = hipEventQuery(rt->staged_done);
    if (state == hipSuccess) {
      rt->staged = 0;
    } else if (state != hipErrorNotReady) {
      return hip_ok(state, "staging event");
    } else if (rt->staged + slot > kStagingBytes) {
      if (hip_ok(hipEventSynchronize(rt->staged_done), "staging wait")) return 1;
      rt->staged = 0;
    }
  }
  slot_out = rt->staging + rt->staged;
  rt->staged += slot;
  return 0;
}

// dst[pairs[2i]] = pairs[2i + 1] for i < count.  The pairs sit in pinned
// host memory that the host filled before queuing the launch; system-scope
// loads read them past the device caches, so a reused staging slot is never
// seen stale.  Indices are distinct (checked on the host), so the stores do
// not race.
__global__ __launch_bounds__(256) void scatter_pairs_kernel(const int32_t* pairs, int32_t* dst,
                                                            int count) {
  int32_t* src = const_cast<int32_t*>(pairs);
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
    const int32_t index = __hip_atomic_load(src + 2 * i, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_SYSTEM);
    const int32_t value = __hip_atomic_load(src + 2 * i + 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_SYSTEM);
    dst[index] = value;
  }
}
}  // namespace

extern "C" int tmc_buf_write_raw_async(tmc_buffer* buf, const void* data, size_t count,
                                       size_t offset) {
  clear_error();
  if (!buf || !data || count == 0 || offset > buf->count || count > buf->count - offset)
    return fail("tmc_buf_write_raw_async: invalid range.");
  tmc_runtime* rt = buf->rt;
  // a captured copy would replay whatever the staging slot holds later
  if (stream_captured(rt))
    return fail("tmc_buf_write_raw_async: not allowed while the runtime stream is captured.");
  const size_t bytes = count * element_bytes(buf->dtype);
  if ((bytes + 255) / 256 * 256 > kStagingBytes) return tmc_buf_write_raw(buf, data, count, offset);
  char* stage = nullptr;
  if (stage_reserve(rt, bytes, stage)) return 1;
  std::memcpy(stage, data, bytes);
  if (hip_ok(hipMemcpyAsync(static_cast<char*>(buf->ptr) + offset * element_bytes(buf->dtype),
                            stage, bytes, hipMemcpyHostToDevice, rt->stream),
             "staged write"))
    return 1;
  return hip_ok(hipEventRecord(rt->staged_done, rt->stream), "staging event");
}

extern "C" int tmc_buf_write_sparse_async(tmc_buffer* buf, const int32_t* pairs, size_t count) {
  clear_error();
  if (!buf || !pairs || count == 0)
    return fail("tmc_buf_write_sparse_async: null buffer or pairs, or no pairs.");
  if (buf->dtype != TMC_I32)
    return fail("tmc_buf_write_sparse_async: the buffer must hold int32 elements.");
  if (count > kStagingBytes / (2 * sizeof(int32_t)))
    return fail("tmc_buf_write_sparse_async: at most 524288 pairs per call.");
  for (size_t i = 0; i < count; ++i) {
    const int32_t index = pairs[2 * i];
    if (index < 0 || (size_t)index >= buf->count || (i > 0 && index <= pairs[2 * i - 2]))
      return fail("tmc_buf_write_sparse_async: indices must increase and lie inside the buffer.");
  }
  tmc_runtime* rt = buf->rt;
  if (stream_captured(rt))
    return fail("tmc_buf_write_sparse_async: not allowed while the runtime stream is captured.");
  const size_t bytes = count * 2 * sizeof(int32_t);
  char* stage = nullptr;
  if (stage_reserve(rt, bytes, stage)) return 1;
  std::memcpy(stage, pairs, bytes);
  const auto* mapped = reinterpret_cast<const int32_t*>(rt->staging_device + (stage - rt->staging));
  const unsigned blocks = (unsigned)std::min<size_t>((count + 255) / 256, 64);
  hipLaunchKernelGGL(scatter_pairs_kernel, dim3(blocks), dim3(256), 0, rt->stream, mapped,
                     static_cast<int32_t*>(buf->ptr), (int)count);
  if (check_launch("scatter_pairs_kernel")) return 1;
  return hip_ok(hipEventRecord(rt->staged_done, rt->stream), "staging event");
}

extern "C" int tmc_buf_copy_async(tmc_buffer* dst, size_t dst_offset, const tmc_buffer* src,
                                  size_t src_offset, size_t count) {
  clear_error();
  if (!dst || !src || dst->rt != src->rt || dst->dtype != src->dtype)
    return fail("tmc_buf_copy_async: buffers of different runtimes or dtypes.");
  if (count == 0 || dst_offset > dst->count || count > dst->count - dst_offset ||
      src_offset > src->count || count > src->count - src_offset)
    return fail("tmc_buf_copy_async: invalid range.");
  const size_t eb = element_bytes(dst->dtype);
  return hip_ok(hipMemcpyAsync(static_cast<char*>(dst->ptr) + dst_offset * eb,
                               static_cast<const char*>(src->ptr) + src_offset * eb, count * eb,
                               hipMemcpyDeviceToDevice, dst->rt->stream),
                "device copy");
}

extern "C" int tmc_buf_read_raw(const tmc_buffer* buf, void* data, size_t count, size_t offset) {
  clear_error();
  if (!buf || !data || offset > buf->count || count > buf->count - offset)
    return fail("tmc_buf_read_raw: invalid range.");
  const size_t eb = element_bytes(buf->dtype);
  if (hip_ok(hipMemcpyAsync(data, static_cast<const char*>(buf->ptr) + offset * eb, count * eb,
                            hipMemcpyDeviceToHost, buf->rt->stream),
             "raw read"))
    return 1;
  return hip_ok(hipStreamSynchronize(buf->rt->stream), "raw read");
}

extern "C" int tmc_buf_read(const tmc_buffer* buf, float* out) {
  clear_error();
  if (!buf || !out) return fail("tmc_buf_read: null argument.");
  std::vector<uint8_t> host(buf->count * element_bytes(buf->dtype));
  if (tmc_buf_read_raw(buf, host.data(), buf->count, 0)) return 1;
  decode_into(host.data(), buf->count, buf->dtype, out);
  return 0;
}

extern "C" int tmc_host_encode(const float* src, size_t count, int dtype, void* dst) {
  clear_error();
  if (!valid_dtype(dtype)) return fail("tmc_host_encode: unknown dtype.");
  if (count && (!src || !dst)) return fail("tmc_host_encode: null argument.");
  encode_into(src, count, dtype, dst);
  return 0;
}

extern "C" int tmc_host_decode(const void* src, size_t count, int dtype, float* dst) {
  clear_error();
  if (!valid_dtype(dtype)) return fail("tmc_host_decode: unknown dtype.");
  if (count && (!src || !dst)) return fail("tmc_host_decode: null argument.");
  decode_into(src, count, dtype, dst);
  return 0;
}

extern "C" size_t tmc_buf_count(const tmc_buffer* buf) { return buf ? buf->count : 0; }
extern "C" int tmc_buf_dtype(const tmc_buffer* buf) { return buf ? buf->dtype : -1; }
extern "C" void* tmc_buf_device_ptr(const tmc_buffer* buf) { return buf ? buf->ptr : nullptr; }

extern "C" void tmc_buf_release(tmc_buffer* buf) {
  if (!buf) return;
  if (buf->owned && buf->ptr) {
    (void)hipStreamSynchronize(buf->rt->stream);
    (void)hipFree(buf->ptr);
  }
  delete buf;
}

extern "C" int tmc_kernel_resolve(tmc_runtime* rt, const char* key, tmc_kernel** out,
                                  int* bindings, int* types, int* writable) {
  clear_error();
  if (!rt || !key || !out) return fail("tmc_kernel_resolve: null argument.");
  if (!rt->available) return fail(rt->init_error);
  std::string name;
  Params params;
  if (!parse_key(key, name, params)) return fail(std::string("Malformed kernel key '") + key + "'.");
  auto kernel = std::make_unique<tmc_kernel>();
  kernel->key = key;
  if (!make_spec(name, params, kernel->spec)) return 1;
  const auto& s = kernel->spec;
  const int n = (int)(s.inputs.size() + s.outputs.size());
  if (bindings) *bindings = n;
  for (int i = 0; i < n; ++i) {
    const bool is_out = i >= (int)s.inputs.size();
    if (types) types[i] = is_out ? s.outputs[i - s.inputs.size()] : s.inputs[i];
    if (writable) writable[i] = is_out ? 1 : 0;
  }
  *out = kernel.release();
  return 0;
}

extern "C" int tmc_kernel_dispatch(const tmc_kernel* kernel, size_t* groups, size_t* threads) {
  if (!kernel) return fail("tmc_kernel_dispatch: null kernel.");
  if (groups) *groups = kernel->spec.groups;
  if (threads) *threads = kernel->spec.threads;
  return 0;
}

extern "C" void tmc_kernel_release(tmc_kernel* kernel) { delete kernel; }

extern "C" int tmc_prepare(tmc_runtime* rt, const tmc_kernel* kernel, tmc_buffer* const* inputs,
                           size_t n_in, tmc_buffer* const* outputs, size_t n_out, size_t groups,
                           size_t threads, const uint32_t* constants, size_t n_constants,
                           tmc_exec** out) {
  clear_error();
  if (!rt || !out) return fail("tmc_prepare: null argument.");
  if (!rt->available) return fail(rt->init_error);
  if (!kernel) return fail("Create a compute pipeline before execution.");
  const size_t binding_count = n_in + n_out + (n_constants ? 1 : 0);
  if (n_in == 0 || n_out == 0 || binding_count > 31 || n_constants > 1024)
    return fail("Invalid buffer binding count or oversized inline constants.");
  if (groups == 0 || groups > std::numeric_limits<uint32_t>::max() || threads == 0 ||
      threads > (size_t)rt->props.maxThreadsPerBlock)
    return fail("Kernel dispatch exceeds device or pipeline limits.");
  const auto& s = kernel->spec;
  if (n_in != s.inputs.size() || n_out != s.outputs.size())
    return fail("Reflection must contain exactly the expected input and output buffers.");
  auto exec = std::make_unique<tmc_exec>();
  exec->rt = rt;
  exec->spec = s;
  for (size_t i = 0; i < n_out; ++i) {
    tmc_buffer* o = outputs[i];
    if (!o || o->rt != rt || std::find(outputs, outputs + i, o) != outputs + i)
      return fail("Outputs must be distinct buffers on the current device.");
    if (o->dtype != s.outputs[i]) return fail("Reflected buffer element type disagrees with TensorIR.");
    if (!s.counts.empty() && o->count < s.counts[n_in + i])
      return fail("Output buffer " + std::to_string(i) + " holds " + std::to_string(o->count) +
                  " elements; the kernel writes " + std::to_string(s.counts[n_in + i]) + ".");
    exec->outputs.push_back(o);
  }
  for (size_t i = 0; i < n_in; ++i) {
    tmc_buffer* b = inputs[i];
    if (!b || b->rt != rt || std::find(outputs, outputs + n_out, b) != outputs + n_out)
      return fail("Input is missing, on another device, or aliases an output.");
    if (b->dtype != s.inputs[i]) return fail("Reflected buffer element type disagrees with TensorIR.");
    if (!s.counts.empty() && b->count < s.counts[i])
      return fail("Input buffer " + std::to_string(i) + " holds " + std::to_string(b->count) +
                  " elements; the kernel reads " + std::to_string(s.counts[i]) + ".");
    exec->ctx.ptrs.push_back(b->ptr);
    exec->ctx.counts.push_back(b->count);
  }
  for (auto* o : exec->outputs) {
    exec->ctx.ptrs.push_back(o->ptr);
    exec->ctx.counts.push_back(o->count);
  }
  if (constants) exec->ctx.constants.assign(constants, constants + n_constants);
  exec->ctx.stream = rt->stream;
  if (s.workspace_bytes) {
    if (hip_ok(hipMalloc(&exec->ctx.workspace, s.workspace_bytes), "workspace allocation")) return 1;
    exec->ctx.workspace_bytes = s.workspace_bytes;
    // A defined starting state for the workspace (filled once, here,
    // outside any captured sequence).
    if (hip_ok(hipMemsetAsync(exec->ctx.workspace, 0, s.workspace_bytes, rt->stream),
               "workspace fill") ||
        hip_ok(hipStreamSynchronize(rt->stream), "workspace fill")) {
      (void)hipFree(exec->ctx.workspace);
      return 1;
    }
  }
  *out = exec.release();
  return 0;
}

extern "C" int tmc_exec_run(tmc_exec* exec, int reset_outputs, double* gpu_us, double* cpu_us) {
  clear_error();
  if (!exec) return fail("tmc_exec_run: null execution.");
  tmc_runtime* rt = exec->rt;
  if (consume_failure(rt)) return 1;
  if (reset_outputs)
    for (auto* o : exec->outputs)
      if (fill_sentinel(o->ptr, o->count, o->dtype, false, rt->stream)) return 1;
  hipEvent_t start = nullptr, stop = nullptr;
  if (gpu_us) {
    if (hip_ok(hipEventCreate(&start), "event") || hip_ok(hipEventCreate(&stop), "event")) return 1;
    (void)hipEventRecord(start, rt->stream);
  }
  const auto t0 = std::chrono::steady_clock::now();
  int rc = exec->spec.launch(exec->ctx);
  if (gpu_us) (void)hipEventRecord(stop, rt->stream);
  const hipError_t sync = hipStreamSynchronize(rt->stream);
  const auto t1 = std::chrono::steady_clock::now();
  if (!rc && sync != hipSuccess) rc = hip_ok(sync, "execution");
  if (cpu_us) *cpu_us = std::chrono::duration<double, std::micro>(t1 - t0).count();
  if (gpu_us) {
    float ms = 0.0f;
    *gpu_us = (!rc && hipEventElapsedTime(&ms, start, stop) == hipSuccess) ? ms * 1000.0 : -1.0;
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
  }
  return rc;
}

extern "C" void tmc_exec_release(tmc_exec* exec) {
  if (!exec) return;
  if (exec->ctx.workspace) {
    (void)hipStreamSynchronize(exec->rt->stream);
    (void)hipFree(exec->ctx.workspace);
  }
  delete exec;
}

extern "C" int tmc_seq_create(tmc_runtime* rt, tmc_exec* const* steps, size_t n, tmc_seq** out) {
  clear_error();
  if (!rt || !out) return fail("tmc_seq_create: null argument.");
  if (n == 0 || !steps) return fail("A prepared region sequence cannot be empty.");
  bool capturable = true;
  for (size_t i = 0; i < n; ++i) {
    if (!steps[i] || !steps[i]->spec.launch) return fail("A region contains an invalid prepared execution.");
    if (steps[i]->rt != rt) return fail("All region steps must use the same runtime stream.");
    capturable = capturable && steps[i]->spec.capturable;
  }
  auto seq = std::make_unique<tmc_seq>();
  seq->rt = rt;
  if (!capturable) {
    for (size_t i = 0; i < n; ++i) seq->eager.emplace_back(steps[i]->spec.launch, steps[i]->ctx);
    *out = seq.release();
    return 0;
  }
  if (hip_ok(hipStreamSynchronize(rt->stream), "sequence capture")) return 1;
  if (hip_ok(hipStreamBeginCapture(rt->stream, hipStreamCaptureModeThreadLocal), "begin capture"))
    return 1;
  int rc = 0;
  for (size_t i = 0; i < n && !rc; ++i) rc = steps[i]->spec.launch(steps[i]->ctx);
  hipGraph_t graph = nullptr;
  const hipError_t end = hipStreamEndCapture(rt->stream, &graph);
  if (rc) {
    if (graph) (void)hipGraphDestroy(graph);
    return 1;
  }
  if (hip_ok(end, "end capture")) return 1;
  seq->graph = graph;
  if (hip_ok(hipGraphInstantiate(&seq->exec, graph, nullptr, nullptr, 0), "graph instantiate")) {
    (void)hipGraphDestroy(graph);
    return 1;
  }
  *out = seq.release();
  return 0;
}

namespace {
// One replay of the sequence on its runtime's stream: the graph, or the
// eager steps in order (stops at the first failing launch).
int replay(tmc_seq* seq) {
  if (seq->exec) return hip_ok(hipGraphLaunch(seq->exec, seq->rt->stream), "graph launch");
  for (const auto& [launch, ctx] : seq->eager)
    if (launch(ctx)) return 1;
  return 0;
}
}  // namespace

extern "C" int tmc_seq_launch(tmc_seq* seq) {
  clear_error();
  if (!seq) return fail("tmc_seq_launch: null sequence.");
  if (consume_failure(seq->rt)) return 1;
  return replay(seq);
}

extern "C" int tmc_seq_run(tmc_seq* seq, double* gpu_us, double* cpu_us) {
  clear_error();
  if (!seq) return fail("tmc_seq_run: null sequence.");
  tmc_runtime* rt = seq->rt;
  if (consume_failure(rt)) return 1;
  hipEvent_t start = nullptr, stop = nullptr;
  if (gpu_us) {
    if (hip_ok(hipEventCreate(&start), "event") || hip_ok(hipEventCreate(&stop), "event")) return 1;
    (void)hipEventRecord(start, rt->stream);
  }
  const auto t0 = std::chrono::steady_clock::now();
  int rc = replay(seq);
  if (gpu_us) (void)hipEventRecord(stop, rt->stream);
  const hipError_t sync = hipStreamSynchronize(rt->stream);
  const auto t1 = std::chrono::steady_clock::now();
  if (!rc && sync != hipSuccess) rc = hip_ok(sync, "sequence execution");
  if (cpu_us) *cpu_us = std::chrono::duration<double, std::micro>(t1 - t0).count();
  if (gpu_us) {
    float ms = 0.0f;
    *gpu_us = (!rc && hipEventElapsedTime(&ms, start, stop) == hipSuccess) ? ms * 1000.0 : -1.0;
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
  }
  return rc;
}

extern "C" void tmc_seq_release(tmc_seq* seq) {
  if (!seq) return;
  (void)hipStreamSynchronize(seq->rt->stream);
  if (seq->exec) (void)hipGraphExecDestroy(seq->exec);
  if (seq->graph) (void)hipGraphDestroy(seq->graph);
  delete seq;
}
