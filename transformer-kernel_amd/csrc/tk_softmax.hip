// Standalone masked softmax over materialised attention scores (HBM-bound).
//
// Row r of a [groups, seq, seq] fp32 score tensor is query i = r % seq of
// group r / seq.  Keys k > i (causal) or k >= key_len[batch] are -inf
// before an fp32 softmax; probabilities are stored as fp16.  Only the valid
// keys of a row are read (a causal row i reads i+1 scores), every key is
// written.  The row is held in registers by LPR lanes (two-pass max/sum on
// registers, one read and one write per element); rows longer than the
// register budget are streamed three times instead.
//
// Numerics follow the baseline (src/torch_transformer_benchmark.py:99-111):
// masked_fill(-inf) then torch.softmax on fp32, cast last.
#include "tk_common.hpp"

namespace tk {
namespace {

constexpr int kBlock = 256;

struct SoftmaxArgs {
  const float* scores;
  f16* probs;
  const int32_t* key_len;
  int64_t rows;
  int seq;
  int heads_per_batch;
  bool causal;
};

__device__ __forceinline__ int valid_keys(const SoftmaxArgs& p, int64_t row) {
  const int i = (int)(row % p.seq);
  int n = p.causal ? i + 1 : p.seq;
  if (p.key_len) {
    const int64_t batch = (row / p.seq) / p.heads_per_batch;
    n = min(n, max(0, (int)p.key_len[batch]));
  }
  return n;
}

// Register-resident rows: each of the LPR lanes holds NV float4 of the row.
template <int LPR, int NV>
__global__ __launch_bounds__(kBlock) void softmax_rows_kernel(SoftmaxArgs p) {
  constexpr int kRowsPerBlock = kBlock / LPR;
  const int lane = threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / LPR;
  if (row >= p.rows) return;
  const int nvalid = valid_keys(p, row);
  const float* sr = p.scores + row * p.seq;
  f16* pr = p.probs + row * p.seq;

  float v[NV][4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c0 = (j * LPR + lane) * 4;
    if (c0 + 3 < nvalid) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(sr + c0);
      v[j][0] = t[0]; v[j][1] = t[1]; v[j][2] = t[2]; v[j][3] = t[3];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[j][e] = (c0 + e < nvalid) ? sr[c0 + e] : -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) mx = fmaxf(mx, v[j][e]);
  }
  mx = group_max<LPR>(mx);
  const float m_use = (mx == -INFINITY) ? 0.f : mx;
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[j][e] = __expf(v[j][e] - m_use);
      sum += v[j][e];
    }
  sum = group_sum<LPR>(sum);
  const float inv = sum > 0.f ? 1.0f / sum : 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c0 = (j * LPR + lane) * 4;
    if (c0 >= p.seq) continue;
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (c0 + e < nvalid) ? v[j][e] * inv : 0.f;
    if (c0 + 3 < p.seq) {
      *reinterpret_cast<f16x4*>(pr + c0) = f16x4{(f16)o[0], (f16)o[1], (f16)o[2], (f16)o[3]};
    } else {
      for (int e = 0; e < 4 && c0 + e < p.seq; ++e) pr[c0 + e] = (f16)o[e];
    }
  }
}

// Long rows: one wave per row, three streaming passes.
__global__ __launch_bounds__(kBlock) void softmax_stream_kernel(SoftmaxArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kBlock / 64) + threadIdx.x / 64;
  if (row >= p.rows) return;
  const int nvalid = valid_keys(p, row);
  const float* sr = p.scores + row * p.seq;
  f16* pr = p.probs + row * p.seq;
  float mx = -INFINITY;
  for (int c = lane; c < nvalid; c += 64) mx = fmaxf(mx, sr[c]);
  mx = group_max<64>(mx);
  const float m_use = (mx == -INFINITY) ? 0.f : mx;
  float sum = 0.f;
  for (int c = lane; c < nvalid; c += 64) sum += __expf(sr[c] - m_use);
  sum = group_sum<64>(sum);
  const float inv = sum > 0.f ? 1.0f / sum : 0.f;
  for (int c = lane; c < p.seq; c += 64) pr[c] = (f16)(c < nvalid ? __expf(sr[c] - m_use) * inv : 0.f);
}

template <int LPR, int NV>
int launch_rows(const SoftmaxArgs& p, hipStream_t st) {
  constexpr int kRowsPerBlock = kBlock / LPR;
  const int64_t grid = (p.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  hipLaunchKernelGGL((softmax_rows_kernel<LPR, NV>), dim3((unsigned)grid), dim3(kBlock), 0, st, p);
  return check_launch("tk_masked_softmax");
}

}  // namespace
}  // namespace tk

using namespace tk;

extern "C" int tk_masked_softmax(const float* scores, tk_half* probs, int64_t groups, int64_t seq,
                                 int causal, const int32_t* key_len, int64_t heads_per_batch,
                                 void* stream) {
  TK_REQUIRE(scores && probs, TK_ERR_ARG, "tk_masked_softmax: null pointer");
  TK_REQUIRE(groups >= 0 && seq >= 0 && seq < (1ll << 30), TK_ERR_ARG, "tk_masked_softmax: bad sizes");
  TK_REQUIRE(key_len == nullptr || heads_per_batch >= 1, TK_ERR_ARG,
             "tk_masked_softmax: key_len needs heads_per_batch >= 1");
  if (groups == 0 || seq == 0) return TK_OK;
  SoftmaxArgs p{};
  p.scores = scores;
  p.probs = reinterpret_cast<f16*>(probs);
  p.key_len = key_len;
  p.rows = groups * seq;
  p.seq = (int)seq;
  p.heads_per_batch = (int)(heads_per_batch < 1 ? 1 : heads_per_batch);
  p.causal = causal != 0;
  hipStream_t st = as_stream(stream);
  const bool vec_ok = seq % 4 == 0 && ((uintptr_t)scores % 16) == 0 && ((uintptr_t)probs % 8) == 0;
  if (vec_ok) {
    if (seq <= 64) return launch_rows<16, 1>(p, st);
    if (seq <= 128) return launch_rows<32, 1>(p, st);
    if (seq <= 256) return launch_rows<64, 1>(p, st);
    if (seq <= 512) return launch_rows<64, 2>(p, st);
    if (seq <= 1024) return launch_rows<64, 4>(p, st);
    if (seq <= 2048) return launch_rows<64, 8>(p, st);
    if (seq <= 4096) return launch_rows<64, 16>(p, st);
  }
  const int64_t grid = (p.rows + 3) / 4;
  hipLaunchKernelGGL(softmax_stream_kernel, dim3((unsigned)grid), dim3(kBlock), 0, st, p);
  return check_launch("tk_masked_softmax");
}
