// FlashAttention-2-style forward for gfx950 (fp16 MFMA, fp32 online softmax).
//
// Per workgroup: BM query rows of one (batch, head), one wave per 32 rows.
// Key/value tiles of 64 keys are staged in LDS (two stages, next tile
// prefetched into registers while the current one is consumed).
//
// Transposed formulation.  Each wave computes S^T = K . Q^T with
// v_mfma_f32_32x32x16_f16 (A operand = K rows from LDS, B operand = the
// wave's Q rows, held in registers for the whole kernel).  In the 32x32
// accumulator layout a lane then holds 16 keys of ONE query row (row =
// lane & 31; lanes l and l^32 hold the two halves), so
//   * the running max / sum of a row need one lane-pair exchange, no LDS;
//   * the rescale of the output accumulator is one scalar per lane;
//   * the fp16 probabilities of 8 consecutive accumulator entries are
//     directly the B operand of O^T = V^T . P^T.
// The keys those 8 entries stand for are {16t+8e2+4g+e10}; V^T is stored in
// LDS with key bits 2 and 3 swapped so that the matching A operand (8 keys
// of one head-dim row d) is one contiguous 16-byte read.
//
// Numerics (src/kernels.py:112-134, src/torch_transformer_benchmark.py:97-111):
// fp32 scores, scale applied in fp32 after Q.K^T (folded with log2(e) into
// one multiply before exp2), -inf masking of future keys, fp32 running
// max/sum, fp16 P for the PV product, fp32 accumulation, one final divide.
#include "tk_common.hpp"

namespace tk {
namespace {

constexpr int kBN = 64;  // keys per tile

// LDS byte offset of the 16-byte chunk `chunk` of row `row` in a tile whose
// rows are RB bytes long.  The gfx950 LDS serves 16-byte-per-lane accesses
// for 16 lanes per cycle from one 256-byte line of 64 banks, so the chunk
// index is XOR-ed with the row's line number (modulo the chunks per row):
// 16 consecutive rows read at one logical chunk then hit 16 distinct 16-byte
// bank groups.
template <int RB>
__device__ __forceinline__ int swz_off(int row, int chunk) {
  if constexpr (RB >= 256) return row * RB + ((chunk ^ (row & 15)) << 4);
  else if constexpr (RB == 128) return row * RB + ((chunk ^ ((row >> 1) & 7)) << 4);
  else if constexpr (RB == 64) return row * RB + ((chunk ^ ((row >> 2) & 3)) << 4);
  else return row * RB + ((chunk ^ ((row >> 3) & 1)) << 4);
}

// Position of key k (0..63 within the tile) in a V^T row: bits 2 and 3 swapped.
__device__ __forceinline__ int vpos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

struct AttnArgs {
  const f16* q;
  const f16* k;
  const f16* v;
  f16* o;
  int64_t qs[3], ks[3], vs[3], os[3];  // element strides for (b, h, s)
  int B, H, S;
  float scale_log2;  // scale * log2(e)
};

template <int HD, int BM, bool CAUSAL>
__global__ __launch_bounds__(BM * 2) void flash_fwd_kernel(AttnArgs p) {
  constexpr int NW = BM / 32;
  constexpr int NT = NW * 64;
  constexpr int KRB = HD * 2;            // K tile row bytes
  constexpr int VRB = kBN * 2;           // V^T tile row bytes (128)
  constexpr int K_CHUNKS = kBN * HD / 8; // 16-byte chunks per K tile
  constexpr int K_LOADS = (K_CHUNKS + NT - 1) / NT;
  constexpr int V_BLOCKS = kBN * HD / 16; // 4 keys x 4 dims micro-blocks
  constexpr int V_LOADS = (V_BLOCKS + NT - 1) / NT;
  constexpr int KSTAGE = kBN * KRB;
  constexpr int VSTAGE = HD * VRB;
  constexpr int DB = (HD + 31) / 32;     // 32-row blocks of the O^T accumulator
  constexpr int KSTEPS = HD / 16;        // k16 steps of S^T = K.Q^T

  __shared__ __attribute__((aligned(16))) char smem[2 * (KSTAGE + VSTAGE)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int BH = p.B * p.H;
  const int n_qt = (p.S + BM - 1) / BM;
  // Heaviest (last) query tiles first; bh fastest so that a head's tiles
  // stay on one XCD (hardware ids are dealt round-robin over 8 XCDs).
  const int id = blockIdx.x;
  const int qt = CAUSAL ? (n_qt - 1 - id / BH) : id / BH;
  const int bh = id % BH;
  const int b = bh / p.H, h = bh % p.H;
  const int q0 = qt * BM;

  const f16* qb = p.q + b * p.qs[0] + h * p.qs[1];
  const f16* kb = p.k + b * p.ks[0] + h * p.ks[1];
  const f16* vb = p.v + b * p.vs[0] + h * p.vs[1];

  const int my_row = q0 + wave * 32 + (lane & 31);
  const int g = lane >> 5;

  // Q^T fragments (B operand): lane supplies Q[row][16*kk + 8*g .. +8].
  f16x8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    if (my_row < p.S)
      qf[kk] = *reinterpret_cast<const f16x8*>(qb + (int64_t)my_row * p.qs[2] + kk * 16 + g * 8);
    else
      qf[kk] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  f32x16 acc_o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[d][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

  const int kv_end = CAUSAL ? min(p.S, q0 + BM) : p.S;
  const int n_kt = (kv_end + kBN - 1) / kBN;

  f16x8 rk[K_LOADS];
  f16x4 rv[V_LOADS][4];

  auto gload = [&](int kt) {
    const int k0 = kt * kBN;
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int idx = tid + i * NT;
      const int key = idx / (HD / 8), ch = idx % (HD / 8);
      if (idx < K_CHUNKS && k0 + key < p.S)
        rk[i] = *reinterpret_cast<const f16x8*>(kb + (int64_t)(k0 + key) * p.ks[2] + ch * 8);
      else
        rk[i] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int idx = tid + i * NT;
      const int kg = idx / (HD / 4), dg = idx % (HD / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = k0 + kg * 4 + e;
        if (idx < V_BLOCKS && key < p.S)
          rv[i][e] = *reinterpret_cast<const f16x4*>(vb + (int64_t)key * p.vs[2] + dg * 4);
        else
          rv[i][e] = f16x4{0, 0, 0, 0};
      }
    }
  };
  auto sstore = [&](int stage) {
    char* ks_ = smem + stage * (KSTAGE + VSTAGE);
    char* vs_ = ks_ + KSTAGE;
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < K_CHUNKS) {
        const int key = idx / (HD / 8), ch = idx % (HD / 8);
        *reinterpret_cast<f16x8*>(ks_ + swz_off<KRB>(key, ch)) = rk[i];
      }
    }
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < V_BLOCKS) {
        const int kg = idx / (HD / 4), dg = idx % (HD / 4);
        const int pos = vpos(kg * 4);  // 4 consecutive keys stay consecutive
#pragma unroll
        for (int e = 0; e < 4; ++e) {  // head-dim row d = 4*dg + e
          const int d = dg * 4 + e;
          f16x4 t = {rv[i][0][e], rv[i][1][e], rv[i][2][e], rv[i][3][e]};
          *reinterpret_cast<f16x4*>(vs_ + swz_off<VRB>(d, pos >> 3) + (pos & 7) * 2) = t;
        }
      }
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();

  const int wave_row_max = q0 + wave * 32 + 31;
  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    const int k0 = kt * kBN;
    if (kt + 1 < n_kt) gload(kt + 1);
    const char* ks_ = smem + cur * (KSTAGE + VSTAGE);
    const char* vs_ = ks_ + KSTAGE;

    if (!CAUSAL || k0 <= wave_row_max) {
      // ---- S^T = K . Q^T : two 32-key blocks ----
      f32x16 sacc[2];
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kb2][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
          const f16x8 kf =
              *reinterpret_cast<const f16x8*>(ks_ + swz_off<KRB>(kb2 * 32 + (lane & 31), 2 * kk + g));
          sacc[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[kk], sacc[kb2], 0, 0, 0);
        }
      }
      // ---- mask, scale, running max ----
      // accumulator entry r of block kb2 is key k0 + 32*kb2 + 8*(r/4) + 4*g + r%4
      const bool need_mask = (k0 + kBN > p.S) || (CAUSAL && k0 + kBN - 1 > q0 + wave * 32);
      float mx = -INFINITY;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float t = sacc[kb2][r] * p.scale_log2;
          if (need_mask) {
            const int key = k0 + kb2 * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key >= p.S || (CAUSAL && key > my_row)) t = -INFINITY;
          }
          sacc[kb2][r] = t;
          mx = fmaxf(mx, t);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run - m_use);
      m_run = m_new;
      float ls = 0.f;
      f16x8 pf[4];
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pv = exp2f(sacc[kb2][hh * 8 + e] - m_use);
            ls += pv;
            pf[kb2 * 2 + hh][e] = (f16)pv;
          }
      l_run = l_run * alpha + ls;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[d][r] *= alpha;
      // ---- O^T += V^T . P^T : four 16-key steps ----
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const int drow = d * 32 + (lane & 31);
          f16x8 vf;
          if (HD % 32 == 0 || drow < HD)
            vf = *reinterpret_cast<const f16x8*>(vs_ + swz_off<VRB>(drow, 2 * t + g));
          else
            vf = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
          acc_o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[t], acc_o[d], 0, 0, 0);
        }
      }
    }

    if (kt + 1 < n_kt) sstore(cur ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane holds O[row][d], d = 32*db + 8*(r/4) + 4*g + r%4 ----
  l_run += __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_run;
  if (my_row < p.S) {
    f16* ob = p.o + b * p.os[0] + h * p.os[1] + (int64_t)my_row * p.os[2];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int dd = d * 32 + 8 * q + 4 * g;
        if (dd < HD) {
          f16x4 t = {(f16)(acc_o[d][4 * q] * inv), (f16)(acc_o[d][4 * q + 1] * inv),
                     (f16)(acc_o[d][4 * q + 2] * inv), (f16)(acc_o[d][4 * q + 3] * inv)};
          *reinterpret_cast<f16x4*>(ob + dd) = t;
        }
      }
  }
}

template <int HD, int BM>
int launch_flash(const AttnArgs& p, bool causal, hipStream_t st) {
  const int64_t n_qt = (p.S + BM - 1) / BM;
  const int64_t grid = n_qt * p.B * p.H;
  if (causal)
    hipLaunchKernelGGL((flash_fwd_kernel<HD, BM, true>), dim3((unsigned)grid), dim3(BM * 2), 0, st, p);
  else
    hipLaunchKernelGGL((flash_fwd_kernel<HD, BM, false>), dim3((unsigned)grid), dim3(BM * 2), 0, st, p);
  return check_launch("tk_flash_attn_fwd");
}

}  // namespace
}  // namespace tk

using namespace tk;

extern "C" int tk_attention_supported(int64_t head_dim) {
  return head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128;
}

extern "C" int tk_flash_attn_fwd(const tk_half* q, const tk_half* k, const tk_half* v, tk_half* out,
                                 int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, const int64_t* o_strides, float scale,
                                 int causal, void* stream) {
  TK_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && o_strides, TK_ERR_ARG,
             "tk_flash_attn_fwd: null pointer");
  TK_REQUIRE(tk_attention_supported(head_dim), TK_ERR_UNSUPPORTED,
             "tk_flash_attn_fwd: head_dim=%lld not in {16, 32, 64, 128}", (long long)head_dim);
  TK_REQUIRE(batch >= 0 && heads >= 0 && seq >= 0 && batch * heads < (1ll << 31) &&
                 seq < (1ll << 30),
             TK_ERR_ARG, "tk_flash_attn_fwd: bad sizes");
  auto al = [](const void* ptr, uintptr_t a) { return ((uintptr_t)ptr % a) == 0; };
  TK_REQUIRE(al(q, 16) && al(k, 16) && al(v, 8) && al(out, 8), TK_ERR_ARG,
             "tk_flash_attn_fwd: q/k need 16-byte, v/out 8-byte alignment");
  for (int i = 0; i < 3; ++i) {
    TK_REQUIRE(q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 4 == 0 &&
                   o_strides[i] % 4 == 0,
               TK_ERR_ARG, "tk_flash_attn_fwd: strides must keep 16-byte (q,k) / 8-byte (v,o) rows");
  }
  if (batch == 0 || heads == 0 || seq == 0) return TK_OK;
  AttnArgs p{};
  p.q = reinterpret_cast<const f16*>(q);
  p.k = reinterpret_cast<const f16*>(k);
  p.v = reinterpret_cast<const f16*>(v);
  p.o = reinterpret_cast<f16*>(out);
  for (int i = 0; i < 3; ++i) {
    p.qs[i] = q_strides[i]; p.ks[i] = k_strides[i]; p.vs[i] = v_strides[i]; p.os[i] = o_strides[i];
  }
  p.B = (int)batch; p.H = (int)heads; p.S = (int)seq;
  p.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = as_stream(stream);
  const bool c = causal != 0;
  // 128-row tiles once there are enough of them to fill the chip; 64 below.
  const bool big = ((seq + 127) / 128) * batch * heads >= 512;
  switch (head_dim) {
    case 16: return big ? launch_flash<16, 128>(p, c, st) : launch_flash<16, 64>(p, c, st);
    case 32: return big ? launch_flash<32, 128>(p, c, st) : launch_flash<32, 64>(p, c, st);
    case 64: return big ? launch_flash<64, 128>(p, c, st) : launch_flash<64, 64>(p, c, st);
    default: return big ? launch_flash<128, 128>(p, c, st) : launch_flash<128, 64>(p, c, st);
  }
}
