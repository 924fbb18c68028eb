// Standalone LayerNorm(+residual add)+cast kernels, HBM-bound.
//
// One row is owned by a group of LPR lanes (16, 32 or 64) of a wave; the
// whole row lives in registers, so the statistics are the exact two-pass
// ones (mean, then mean of squared deviations: population variance) with one
// HBM read and one write per element.  Row reductions are butterfly shuffles
// inside the lane group -- no LDS, no __syncthreads.
//
// Numerics follow src/fused_kernels.py:80-161: fp32 add, fp32 statistics,
// y = (s - mean) * rstd * w + b, cast last.
//
// Launches whose fp32 input exceeds half the 256 MB Infinity Cache use
// non-temporal loads and stores for the 16-byte row vectors (each element is
// touched once): ln_cast fp32 -> fp16 at 32768 x 2048 (C4) 87 -> 75 us per
// launch in a same-box A/B of the whole forward.  Smaller launches keep
// ordinary accesses: their output is read back from the cache by the next
// GEMM, and non-temporal stores made C2's forward 4 % slower.
#include "tk_common.hpp"

namespace tk {
namespace {

constexpr int kBlock = 256;

template <bool NT, typename V>
__device__ __forceinline__ V ld(const V* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT, typename V>
__device__ __forceinline__ void st(V* p, V v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <typename T, bool NT = false>
struct Vec;
template <bool NT>
struct Vec<float, NT> {
  static __device__ __forceinline__ void load4(const float* p, float* v) {
    f32x4 t = ld<NT>(reinterpret_cast<const f32x4*>(p));
    v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
  }
  static __device__ __forceinline__ void store4(float* p, const float* v) {
    f32x4 t = {v[0], v[1], v[2], v[3]};
    st<NT>(reinterpret_cast<f32x4*>(p), t);
  }
  static __device__ __forceinline__ float load1(const float* p) { return *p; }
  static __device__ __forceinline__ void store1(float* p, float v) { *p = v; }
};
template <bool NT>
struct Vec<f16, NT> {
  static __device__ __forceinline__ void load4(const f16* p, float* v) {
    f16x4 t = ld<NT>(reinterpret_cast<const f16x4*>(p));
    v[0] = (float)t[0]; v[1] = (float)t[1]; v[2] = (float)t[2]; v[3] = (float)t[3];
  }
  static __device__ __forceinline__ void store4(f16* p, const float* v) {
    f16x4 t = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    st<NT>(reinterpret_cast<f16x4*>(p), t);
  }
  static __device__ __forceinline__ float load1(const f16* p) { return (float)*p; }
  static __device__ __forceinline__ void store1(f16* p, float v) { *p = (f16)v; }
};

// HAS_Y: s = x + y (residual add, in fp32) else s = x.  The sum is stored in
// x's type XT (src/fused_kernels.py:216,143-147: s = x + y in x's dtype); the
// statistics use the fp32 sum before that rounding.  row_valid (nullable): an
// invalid row's normalised output is written as zeros.
template <int LPR, int NV, int VW, bool HAS_Y, typename XT, typename YT, typename OT, bool NT>
__global__ __launch_bounds__(kBlock) void ln_rows_kernel(
    const XT* x, const YT* __restrict__ y, const float* __restrict__ w,
    const float* __restrict__ b, XT* sum_out, OT* __restrict__ out, int64_t rows,
    int cols, float eps, const uint8_t* __restrict__ row_valid) {
  constexpr int kRowsPerBlock = kBlock / LPR;
  const int lane = threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / LPR;
  if (row >= rows) return;

  const XT* xr = x + row * cols;
  float s[NV * VW];

#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c0 = (v * LPR + lane) * VW;
    if constexpr (VW == 4) {
      if (c0 < cols) {
        Vec<XT, NT>::load4(xr + c0, &s[v * 4]);
        if constexpr (HAS_Y) {
          float t[4];
          Vec<YT, NT>::load4(y + row * cols + c0, t);
#pragma unroll
          for (int e = 0; e < 4; ++e) s[v * 4 + e] += t[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) s[v * 4 + e] = 0.f;
      }
    } else {
      if (c0 < cols) {
        s[v] = Vec<XT>::load1(xr + c0);
        if constexpr (HAS_Y) s[v] += Vec<YT>::load1(y + row * cols + c0);
      } else {
        s[v] = 0.f;
      }
    }
  }

  if (HAS_Y && sum_out != nullptr) {
    XT* sr = sum_out + row * cols;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int c0 = (v * LPR + lane) * VW;
      if (c0 < cols) {
        if constexpr (VW == 4) Vec<XT, NT>::store4(sr + c0, &s[v * 4]);
        else Vec<XT>::store1(sr + c0, s[v]);
      }
    }
  }

  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < NV * VW; ++i) acc += s[i];
  const float mean = group_sum<LPR>(acc) / (float)cols;

  acc = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c0 = (v * LPR + lane) * VW;
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      const float d = (c0 + e < cols) ? s[v * VW + e] - mean : 0.f;
      s[v * VW + e] = d;
      acc += d * d;
    }
  }
  const float var = group_sum<LPR>(acc) / (float)cols;
  float rstd = 1.0f / sqrtf(var + eps);
  // padded row: (s - mean) * 0 * w + 0 written as exact zeros
  const bool keep = row_valid == nullptr || row_valid[row] != 0;
  if (!keep) rstd = 0.f;

  OT* orow = out + row * cols;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c0 = (v * LPR + lane) * VW;
    if (c0 < cols) {
      if constexpr (VW == 4) {
        const f32x4 wv = *reinterpret_cast<const f32x4*>(w + c0);
        const f32x4 bv = *reinterpret_cast<const f32x4*>(b + c0);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = keep ? s[v * 4 + e] * rstd * wv[e] + bv[e] : 0.f;
        Vec<OT, NT>::store4(orow + c0, o);
      } else {
        Vec<OT>::store1(orow + c0, keep ? s[v] * rstd * w[c0] + b[c0] : 0.f);
      }
    }
  }
}

constexpr int64_t kStreamBytes = 128ll << 20;  // fp32 input size from which the accesses are non-temporal

template <int LPR, int NV, int VW, bool HAS_Y, typename XT, typename YT, typename OT>
int launch_rows(const XT* x, const YT* y, const float* w, const float* b, XT* sum_out,
                OT* out, int64_t rows, int cols, float eps, const uint8_t* row_valid, hipStream_t st) {
  constexpr int kRowsPerBlock = kBlock / LPR;
  const int64_t grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (VW == 4 && rows * cols * 4 >= kStreamBytes)
    hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, VW, HAS_Y, XT, YT, OT, true>), dim3((unsigned)grid),
                       dim3(kBlock), 0, st, x, y, w, b, sum_out, out, rows, cols, eps, row_valid);
  else
    hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, VW, HAS_Y, XT, YT, OT, false>), dim3((unsigned)grid),
                       dim3(kBlock), 0, st, x, y, w, b, sum_out, out, rows, cols, eps, row_valid);
  return check_launch("layernorm");
}

// Picks lanes-per-row and register-vector count for `cols`.
template <bool HAS_Y, typename XT, typename YT, typename OT>
int dispatch(const XT* x, const YT* y, const float* w, const float* b, XT* sum_out,
             OT* out, int64_t rows, int cols, float eps, const uint8_t* row_valid, hipStream_t st) {
#define TK_LN(LPR, NV, VW) \
  return launch_rows<LPR, NV, VW, HAS_Y, XT, YT, OT>(x, y, w, b, sum_out, out, rows, cols, eps, row_valid, st)
  // 4-wide vector path needs cols % 4 == 0 and rows aligned to 4 elements
  // (16 bytes for fp32 rows, 8 for fp16); anything else takes the scalar path.
  auto al = [](const void* p, uintptr_t a) { return p == nullptr || ((uintptr_t)p % a) == 0; };
  const bool vec_ok = cols % 4 == 0 && al(x, sizeof(XT) * 4) && al(w, 16) && al(b, 16) &&
                      al(sum_out, sizeof(XT) * 4) && al(y, sizeof(YT) * 4) && al(out, sizeof(OT) * 4);
  if (vec_ok) {
    if (cols <= 64) TK_LN(16, 1, 4);
    if (cols <= 128) TK_LN(32, 1, 4);
    const int nv = (cols + 255) / 256;
    if (nv <= 1) TK_LN(64, 1, 4);
    if (nv <= 2) TK_LN(64, 2, 4);
    if (nv <= 3) TK_LN(64, 3, 4);
    if (nv <= 4) TK_LN(64, 4, 4);
    if (nv <= 6) TK_LN(64, 6, 4);
    if (nv <= 8) TK_LN(64, 8, 4);
    if (nv <= 16) TK_LN(64, 16, 4);
    TK_LN(64, 32, 4);
  }
  const int nv = (cols + 63) / 64;
  if (nv <= 1) TK_LN(64, 1, 1);
  if (nv <= 2) TK_LN(64, 2, 1);
  if (nv <= 4) TK_LN(64, 4, 1);
  if (nv <= 8) TK_LN(64, 8, 1);
  if (nv <= 16) TK_LN(64, 16, 1);
  if (nv <= 32) TK_LN(64, 32, 1);
  if (nv <= 64) TK_LN(64, 64, 1);
  TK_LN(64, 128, 1);
#undef TK_LN
}

constexpr int64_t kMaxCols = 8192;

}  // namespace
}  // namespace tk

using namespace tk;

extern "C" int tk_ln_cast(const float* x, const float* w, const float* b, void* out,
                          int out_dtype, int64_t rows, int64_t cols, float eps,
                          const uint8_t* row_valid, void* stream) {
  TK_REQUIRE(x && w && b && out, TK_ERR_ARG, "tk_ln_cast: null pointer");
  TK_REQUIRE(rows >= 0 && cols >= 1 && cols <= kMaxCols, TK_ERR_ARG,
             "tk_ln_cast: rows=%lld cols=%lld outside [0, inf) x [1, %lld]", (long long)rows,
             (long long)cols, (long long)kMaxCols);
  TK_REQUIRE(out_dtype == TK_F16 || out_dtype == TK_F32, TK_ERR_ARG,
             "tk_ln_cast: bad out_dtype %d", out_dtype);
  if (rows == 0) return TK_OK;
  hipStream_t st = as_stream(stream);
  const int c = (int)cols;
  if (out_dtype == TK_F16)
    return dispatch<false, float, float, f16>(x, nullptr, w, b, nullptr, (f16*)out, rows, c, eps, row_valid, st);
  return dispatch<false, float, float, float>(x, nullptr, w, b, nullptr, (float*)out, rows, c, eps, row_valid,
                                              st);
}

namespace {
template <typename XT>
int add_ln_x(const XT* x, const void* y, int y_dtype, const float* w, const float* b, XT* sum_out,
             void* h_out, int h_dtype, int64_t rows, int c, float eps, hipStream_t st) {
  if (y_dtype == TK_F16) {
    if (h_dtype == TK_F16)
      return dispatch<true, XT, f16, f16>(x, (const f16*)y, w, b, sum_out, (f16*)h_out, rows, c, eps, nullptr, st);
    return dispatch<true, XT, f16, float>(x, (const f16*)y, w, b, sum_out, (float*)h_out, rows, c, eps, nullptr,
                                          st);
  }
  if (h_dtype == TK_F16)
    return dispatch<true, XT, float, f16>(x, (const float*)y, w, b, sum_out, (f16*)h_out, rows, c, eps, nullptr,
                                          st);
  return dispatch<true, XT, float, float>(x, (const float*)y, w, b, sum_out, (float*)h_out, rows, c, eps,
                                          nullptr, st);
}
}  // namespace

extern "C" int tk_add_ln_cast(const void* x, int x_dtype, const void* y, int y_dtype, const float* w,
                              const float* b, void* sum_out, void* h_out, int h_dtype,
                              int64_t rows, int64_t cols, float eps, void* stream) {
  TK_REQUIRE(x && y && w && b && h_out, TK_ERR_ARG, "tk_add_ln_cast: null pointer");
  TK_REQUIRE(rows >= 0 && cols >= 1 && cols <= kMaxCols, TK_ERR_ARG,
             "tk_add_ln_cast: rows=%lld cols=%lld outside [0, inf) x [1, %lld]",
             (long long)rows, (long long)cols, (long long)kMaxCols);
  TK_REQUIRE((x_dtype == TK_F16 || x_dtype == TK_F32) && (y_dtype == TK_F16 || y_dtype == TK_F32) &&
                 (h_dtype == TK_F16 || h_dtype == TK_F32),
             TK_ERR_ARG, "tk_add_ln_cast: bad dtype (x=%d, y=%d, h=%d)", x_dtype, y_dtype, h_dtype);
  if (rows == 0) return TK_OK;
  hipStream_t st = as_stream(stream);
  const int c = (int)cols;
  if (x_dtype == TK_F16)
    return add_ln_x<f16>((const f16*)x, y, y_dtype, w, b, (f16*)sum_out, h_out, h_dtype, rows, c, eps, st);
  return add_ln_x<float>((const float*)x, y, y_dtype, w, b, (float*)sum_out, h_out, h_dtype, rows, c, eps, st);
}
