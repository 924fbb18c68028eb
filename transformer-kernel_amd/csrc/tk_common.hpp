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

typedef __attribute__((address_space(3))) char lds_char;
typedef __fp16 hf16x2 __attribute__((ext_vector_type(2)));  // operand type of the fdot2 builtin
typedef __fp16 tr_f16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) tr_f16x4 lds_tr_f16x4;

// Max / sum over the lane pair (l, l^32) that holds one row of a 32x32 MFMA
// accumulator (lanes l and l^32 hold the two halves of column l & 31).
// v_permlane32_swap of a register with itself leaves, in every lane, its own
// value in one half of the result and the partner's in the other, so a
// symmetric op over both halves is the pair reduction -- two VALU ops, no
// LDS round trip.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One 16-byte-per-lane global -> LDS copy of a wave (global_load_lds_dwordx4:
// lane l's 16 bytes land at lds_addr + 16*l; lds_addr wave-uniform).  Issued
// as inline assembly so that the compiler's wait insertion, which cannot tell
// a kernel's LDS ring slots apart, does not put a vmcnt wait in front of
// every later LDS read; the kernels wait for their copies themselves (vmcnt
// before each workgroup barrier).  M0 is saved and restored.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gptr), "s"(lds_addr)
      : "memory");
}

// s_waitcnt with vmcnt <= N, other counters unconstrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the memory fence of __syncthreads() (which
// waits for every outstanding vector-memory op, i.e. drains all in-flight
// tile copies).  The empty asm statements keep the compiler from moving LDS
// accesses across it; the direct-copy loop orders the copies itself with
// wait_vmcnt, and every fragment read has completed before the MFMA that
// consumes it was issued.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}


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

// GELU with the exact (erf) form, x*Phi(x) = 0.5*x*(1+erf(x/sqrt(2))), as
// F.gelu(approximate="none").  For either sign of x, GELU(x) = max(x, 0) - r(a)
// with a = |x| and r(a) = a*Phi(-a) >= 0 (x - x*Phi(-x) for x >= 0, x*Phi(x)
// for x < 0), with no 1+erf cancellation.  log2 Phi(-a) is smooth and concave,
// so r(a) = a * 2^P(a) with P of degree 5: P(0) = -1 exactly and c1..c5
// minimise max |a*2^P(a) - r(a)| on [0, 10] (a linear program over a dense
// grid, fit_gelu.py beside this file).  The leading coefficient is negative,
// so beyond the fitted range 2^P keeps falling and underflows to 0 (the
// result is then max(x, 0) for any finite x).  Evaluated in fp32, |GELU
// error| <= 7.2e-7 on [-12, 12], rounding of the result included; near 0 the
// relative error is below 1e-6.  6 VALU ops (5 FMAs and the final FMA) and
// one v_exp_f32, no select.
__device__ __forceinline__ float gelu_erf(float x) {
  const float a = fabsf(x);
  float p = fmaf(-4.889519769e-04f, a, 7.205033675e-03f);
  p = fmaf(p, a, -5.216291174e-02f);
  p = fmaf(p, a, -4.595786631e-01f);
  p = fmaf(p, a, -1.151006579e+00f);
  p = fmaf(p, a, -1.0f);
  return fmaf(-a, __builtin_amdgcn_exp2f(p), fmaxf(x, 0.0f));
}

}  // namespace tk
