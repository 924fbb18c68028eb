// One-key-tile attention (S <= 64 keys, head_dim <= 64) on operands already
// in LDS and registers, shared by the single-tile flash kernel
// (tk_attention.hip) and the fused QKV-projection + attention kernel
// (tk_gemm.hip), so both compute the same arithmetic in the same order.
//
// Layouts (one tile = 64 rows of RB = 2 * head_dim bytes):
//   K tile: row-major, 16-byte chunks XOR-swizzled by swz_off<RB>;
//   V tile: row-major, chunk XOR vswz<RB>(row) for the transposed reads;
//   Q: this lane's query row as B operands, qf[kk] = Q[row][16kk + 8g .. +8]
//      with g = lane >> 5.
// Numerics (src/kernels.py:112-134, src/torch_transformer_benchmark.py:97-111):
// fp32 scores S^T = K . Q^T, -inf for masked keys, the exact row max, exp2
// with scale * log2(e) folded into one FMA, fp16 P, fp32 row sums of the
// fp16 P, O^T = V^T . P^T in fp32, one final divide, fp16 output.
#pragma once
#include "tk_common.hpp"

namespace tk {
namespace {

// LDS byte offset of the 16-byte chunk `chunk` of row `row` in a K tile
// whose rows are RB bytes long.  The gfx950 LDS serves 16-byte-per-lane
// accesses for 16 lanes per cycle from one 256-byte line of 64 banks, so the
// chunk index is XOR-ed with the row's line number (modulo the chunks per
// row): 16 consecutive rows read at one logical chunk then hit 16 distinct
// 16-byte bank groups.
template <int RB>
__device__ __forceinline__ int swz_off(int row, int chunk) {
  if constexpr (RB >= 256) return row * RB + ((chunk ^ (row & 15)) << 4);
  else if constexpr (RB == 128) return row * RB + ((chunk ^ ((row >> 1) & 7)) << 4);
  else if constexpr (RB == 64) return row * RB + ((chunk ^ ((row >> 2) & 3)) << 4);
  else return row * RB + ((chunk ^ ((row >> 3) & 1)) << 4);
}

// Chunk XOR of a V tile row for the transposed reads: the four rows a
// half-wave reads (r0..r0+3, r0 % 4 == 0) must put the 32 bytes each of them
// contributes on distinct banks.  Rows of 64 or 32 bytes already do.
template <int RB>
__device__ __forceinline__ int vswz(int row) {
  if constexpr (RB >= 256) return 4 * (row & 3);
  else if constexpr (RB == 128) return 4 * ((row >> 1) & 1);
  else return 0;
}

// Attention of one 32-row query block (this wave) over one key tile.
// my_row: this lane's query row (lane & 31 of the wave's block) within the
// sequence; S: keys (and query rows) of the sequence; kbits (KMASK): bit j
// set when key j is valid; cs: scale * log2(e); O row r of the sequence is
// obase + r * ostride (only rows < S are written).
template <int HD, bool CAUSAL, bool KMASK>
__device__ __forceinline__ void attend_one_tile(const char* ks_, const char* vs_, const f16x8 (&qf)[HD / 16],
                                                int my_row, int S, uint64_t kbits, float cs, f16* obase,
                                                int64_t ostride) {
  constexpr int RB = HD * 2;
  constexpr int DB = (HD + 31) / 32;  // 32-row blocks of the O^T accumulator
  constexpr int KSTEPS = HD / 16;     // k16 steps of S^T = K.Q^T
  constexpr int NS = 2 * KSTEPS;      // S^T MFMAs
  constexpr int NP = 4 * DB;          // O^T MFMAs
  static_assert(HD <= 64, "one key tile holds head_dim <= 64");
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5;

  // ---- S^T = K . Q^T: entry r of block kb2 is key 32*kb2 + 8*(r/4) + 4*g + r%4 ----
  f32x16 s[2];
#pragma unroll
  for (int c = 0; c < NS; ++c) {
    const int kb2 = c / KSTEPS, kk = c % KSTEPS;
    const f16x8 kf = *reinterpret_cast<const f16x8*>(ks_ + swz_off<RB>(kb2 * 32 + (lane & 31), 2 * kk + g));
    s[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[kk], kk == 0 ? f32x16{} : s[kb2], 0, 0, 0);
  }
  float mx = -INFINITY;
  const uint64_t kb64 = kbits >> (4 * g);
#pragma unroll
  for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = kb2 * 32 + 8 * (r >> 2) + (r & 3);
      const int key = j + 4 * g;
      if (key >= S || (CAUSAL && key > my_row) || (KMASK && ((kb64 >> j) & 1) == 0)) s[kb2][r] = -INFINITY;
      mx = fmaxf(mx, s[kb2][r]);
    }
  mx = pair_max(mx);
  const float m_tile = mx * cs;  // cs > 0: max(s)*cs == max(s*cs)
  const float m_use = m_tile == -INFINITY ? 0.f : m_tile;

  // ---- P in fp16 (8 consecutive entries = one B operand) and its row sum ----
  f16x8 pf[4];
  float ls = 0.f;
#pragma unroll
  for (int e = 0; e < 32; e += 2) {
    const float p0 = __builtin_amdgcn_exp2f(fmaf(s[e >> 4][e & 15], cs, -m_use));
    const float p1 = __builtin_amdgcn_exp2f(fmaf(s[(e + 1) >> 4][(e + 1) & 15], cs, -m_use));
    const f16x2 hp = {(f16)p0, (f16)p1};
    pf[e >> 3][e & 7] = hp[0];
    pf[e >> 3][(e & 7) + 1] = hp[1];
    ls += p0;  // row sum of the fp32 exponentials, in entry order (as flash_dma_body)
    ls += p1;
  }

  // ---- O^T = V^T . P^T; V^T operands by transposed LDS reads ----
  // lane = 16*q + s; read r (0/1) covers keys 16t + 8r + 4*(q >> 1) + (s >> 2)
  // and head-dim columns 32*db + 16*(q & 1) + 4*(s & 3).
  int v_rd[2][DB];
  {
    const int tq = lane >> 4, ts = lane & 15;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const int row = 8 * r + 4 * (tq >> 1) + (ts >> 2);
        const int col = 32 * d + (HD >= 32 ? 16 * (tq & 1) : 0) + 4 * (ts & 3);  // HD 16: lanes >= 16 are zeroed
        v_rd[r][d] = row * RB + (((col >> 3) ^ vswz<RB>(row)) << 4) + (col & 7) * 2;
      }
  }
  const bool d_ok = HD % 32 == 0 || (lane & 31) < HD;
  f32x16 acc_o[DB];
#pragma unroll
  for (int c = 0; c < NP; ++c) {
    const int t = c / DB, d = c % DB;
    const lds_char* base = (const lds_char*)(vs_ + t * 16 * RB);
    const tr_f16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[0][d]));
    const tr_f16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[1][d]));
    f16x8 vf = __builtin_shufflevector(__builtin_bit_cast(f16x4, lo), __builtin_bit_cast(f16x4, hi), 0, 1, 2, 3, 4,
                                       5, 6, 7);
    if (!d_ok) vf = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    acc_o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[t], t == 0 ? f32x16{} : acc_o[d], 0, 0, 0);
  }

  // ---- normalise and store: lane holds O[row][d], d = 32*db + 8*(r/4) + 4*g + r%4 ----
  const float inv = 1.0f / pair_sum(ls);
  if (my_row < S) {
    f16* orow = obase + (int64_t)my_row * ostride;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int dd = d * 32 + 8 * q + 4 * g;
        if (dd < HD) {
          f16x4 t = {(f16)(acc_o[d][4 * q] * inv), (f16)(acc_o[d][4 * q + 1] * inv),
                     (f16)(acc_o[d][4 * q + 2] * inv), (f16)(acc_o[d][4 * q + 3] * inv)};
          *reinterpret_cast<f16x4*>(orow + dd) = t;
        }
      }
  }
}

}  // namespace
}  // namespace tk
