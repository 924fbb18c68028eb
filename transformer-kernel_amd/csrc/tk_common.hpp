// Shared device/host helpers for the gfx950 kernels of libtkmi.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "tkmi.h"

namespace tk {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors --
// Per-thread status text behind tk_last_error_string().
void set_error(const char* fmt, ...);
void clear_error();
const char* last_error();

// Returns TK_ERR_HIP (and records the text) if the launch just issued failed.
int check_launch(const char* what);

#define TK_REQUIRE(cond, code, ...)      \
  do {                                   \
    if (!(cond)) {                       \
      ::tk::set_error(__VA_ARGS__);      \
      return (code);                     \
    }                                    \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------- wave reductions --
// Butterfly sum over groups of `width` lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WIDTH);
  return v;
}

template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, WIDTH));
  return v;
}

// Exact GELU, 0.5*x*(1+erf(x/sqrt(2))), using the device erff.
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

}  // namespace tk
