// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/tmc_hip.h"
#include "../../include/tmc_bench.h"

namespace tmc {

void set_error(const std::string& message);
void clear_error();

inline hipStream_t as_stream(void* stream) { return reinterpret_cast<hipStream_t>(stream); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Returns 0, or sets the error text and returns 1.
int check_launch(const char* what);

inline int fail(const std::string& message) {
  set_error(message);
  return 1;
}

}  // namespace tmc

#define TMC_REQUIRE(cond, msg) \
  do {                         \
    if (!(cond)) return ::tmc::fail(msg); \
  } while (0)
