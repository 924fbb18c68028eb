// Whole-forward kernel for narrow models (d_model = ffn_dim = 128, attention
// width 128, S <= 128): the reference's own config 1 and most of its
// appendix shapes, where the layer-by-layer path is ~36 launches of a few
// microseconds each per forward.
//
// One workgroup runs the complete forward of one sequence, all layers,
// without touching HBM between kernels.  8 waves (two per SIMD, so one
// wave's LDS, L2 and barrier latency overlaps the other's MFMAs; 4 waves
// when S <= 32 leaves a single row block):
//   * the fp32 residual stream x stays in registers for the whole forward:
//     wave w owns columns [32c, 32c+32), c = w & 3, of the row blocks
//     (w >> 2) and (w >> 2) + 2, in the 32x32 MFMA accumulator layout of C^T
//     (lane l holds 4 consecutive columns of row 32*mb + (l & 31) per 4
//     registers), so the out-projection and FFN-down products accumulate
//     straight into it;
//   * LayerNorm row statistics are combined across the 4 column waves of a
//     row through a small LDS table (exact two-pass mean / variance);
//   * the GEMMs compute C^T = W . A^T on v_mfma_f32_32x32x16_f16: the A
//     operand is a weight fragment (16 bytes per lane, read from L2 one phase
//     ahead of its use, the QKV blocks one block ahead), the B operand an
//     activation fragment from a chunk-swizzled LDS tile (h, Q, K, ctx, u);
//   * attention: one item per (head, 32-row query block), items dealt to
//     the waves heaviest first; S^T = K . Q^T per 32-key block with FA-2
//     online softmax across the at most 4 key blocks (fp32 scores, -inf
//     masking, running max, exp2 with the scale folded, fp16 P, row sums of
//     the fp16 P, O rescaled when the max grows), O^T = V^T . P^T with V^T
//     from ds_read_b64_tr_b16 reads of the row-major V tile.
// Numerics are those of the layer-by-layer path (src/optimized.py:488-554;
// src/kernels.py:112-134): fp16 operands, fp32 accumulation, residual and
// statistics, bias/GELU/residual in fp32 before each fp16 rounding.
#include "tk_common.hpp"

#include <algorithm>
#include <mutex>

namespace tk {
namespace {

constexpr int kMaxRows = 128;  // S <= 128: four 32-row blocks
constexpr int kPitch = 256;    // bytes per LDS tile row (128 fp16 columns)
constexpr int kTile = kMaxRows * kPitch;

struct SmallArgs {
  const float* x;
  float* out;
  const f16* w_qkv;  // [L][3*DP][D]
  const float* b_qkv;
  const f16* w_o;  // [L][D][DP]
  const float* b_o;
  const f16* w_1;  // [L][F][D]
  const float* b_1;
  const f16* w_2;  // [L][D][F]
  const float* b_2;
  const float* n1_w;  // [L][D]
  const float* n1_b;
  const float* n2_w;
  const float* n2_b;
  const float* nf_w;  // [D]
  const float* nf_b;
  float n1_eps, n2_eps, nf_eps;
  float scale_log2;  // attention scale * log2(e)
  int S, L, H;
  // Split sequences (one 32-row block per workgroup): batch size, K/V hand-off slots
  // [batch][layer][4 blocks][K rows | V rows] and their consumer counts, same index.
  int B;
  char* ws;
  unsigned* flags;
};

// Byte offset of 16-byte chunk c of row r in an activation tile: the chunk
// index is XOR-ed with r mod 16, so the 32 rows of a fragment read (one
// chunk each) and the row writes hit distinct banks.
__device__ __forceinline__ int act_off(int r, int c) { return r * kPitch + ((c ^ (r & 15)) << 4); }
// V tile: chunk XOR 4*(r mod 4), the layout the transposed reads need (the
// four rows a 16-lane group reads put their bytes on distinct banks).
__device__ __forceinline__ int v_off(int r, int c) { return r * kPitch + ((c ^ (4 * (r & 3))) << 4); }

// Workgroup barrier for LDS hand-offs: this wave's LDS accesses complete
// (lgkmcnt 0), then s_barrier.  __syncthreads() would also wait for every
// outstanding global load -- the weight fragments issued a phase ahead.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Bound on a split block's wait for an earlier block's K/V (each try sleeps ~128 cycles): every
// block of a split launch is resident (the host splits only when batch x blocks <= CUs) and the
// earlier blocks of a sequence never wait on later ones, so it is never reached in a working
// launch; if it is, the block's output rows are NaN instead of a hang.
constexpr unsigned kSpinLimit = 1u << 20;
constexpr int kSlotBytes = 2 * 32 * kPitch;  // K then V rows of one 32-row block: 16 KB

// SPLIT (causal, S > 32): workgroup j * batch + b runs the 32-row block j of sequence b with 4
// waves; after each layer's QKV it hands its K and V rows to the later blocks of the sequence
// through p.ws and takes those of the earlier blocks (causal attention needs keys <= its rows
// only).  Every other phase is row-local.  The ids are j-major, so the blocks a workgroup waits
// for were dispatched before it, and with a batch that is a multiple of 8 a sequence's blocks
// share an XCD (ids are dealt round-robin over the 8 XCDs) and its L2.
template <int D, int DP, int F, int HDP, bool CAUSAL, bool SPLIT>
__global__ __launch_bounds__(512, 1) void small_forward_kernel(SmallArgs p) {
  static_assert(!SPLIT || CAUSAL, "split sequences: causal attention only");
  static_assert(D == 128 && DP == 128 && F == 128, "one width: 4 column waves x 32 columns");
  static_assert(HDP == 16 || HDP == 32 || HDP == 64 || HDP == 128, "head dims with an MFMA k-step");
  constexpr int KD = D / 16, KP = DP / 16, KF = F / 16;  // k-steps
  constexpr int NQ = 3 * DP / 32 / 4;                      // QKV n-blocks per column wave
  constexpr int HK = HDP / 16;                             // k-steps of one head
  constexpr int DB = (HDP + 31) / 32;                      // 32-row blocks of O^T

  // Per-layer vectors, staged in LDS one layer ahead (double-buffered):
  // b_qkv | b_o | b_1 | b_2 | n1_w | n1_b | n2_w | n2_b, then the final norm.
  constexpr int V_BO = 3 * DP, V_B1 = V_BO + D, V_B2 = V_B1 + F, V_N1W = V_B2 + D, V_N1B = V_N1W + D,
                V_N2W = V_N1B + D, V_N2B = V_N2W + D, VEC = V_N2B + D;
  static_assert(3 * DP <= 512, "b_qkv: at most two elements per thread of 256");

  __shared__ __attribute__((aligned(16))) char smem[4 * kTile + 2 * 4 * kMaxRows * 4 + (2 * VEC + 2 * D) * 4 + 16];
  char* Ht = smem;                // h (LayerNorm output) / ctx
  char* Qt = smem + kTile;        // Q / u
  char* Kt = smem + 2 * kTile;    // K
  char* Vt = smem + 3 * kTile;    // V
  float* stats = reinterpret_cast<float*>(smem + 4 * kTile);  // [2][4 column waves][128 rows]
  float* vecs = stats + 2 * 4 * kMaxRows;                     // [2][VEC], then nf_w, nf_b
  int* lost = reinterpret_cast<int*>(vecs + 2 * VEC + 2 * D);  // split: an earlier block was not seen

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wc = w & 3;   // column block: columns [32 wc, 32 wc + 32) of every 128-wide product
  const int rh = w >> 2;  // row blocks rh and rh + 2
  // Lane coordinates.  refresh() passes them through an empty asm at the
  // start of each phase, so the LDS addresses derived from them (one per
  // swizzled 16-byte chunk) are recomputed per phase instead of being hoisted
  // out of the layer loop and held in registers for the whole forward.
  int g = lane >> 5;
  int rl = lane & 31;
  int tq = lane >> 4, ts = lane & 15;
  auto refresh = [&]() { asm volatile("" : "+v"(g), "+v"(rl), "+v"(tq), "+v"(ts)); };
  const int S = p.S;
  const int MB = (S + 31) >> 5;
  const int jb = SPLIT ? (int)(blockIdx.x / (unsigned)p.B) : 0;  // split: this workgroup's row block
  const int64_t b = SPLIT ? (int64_t)(blockIdx.x % (unsigned)p.B) : (int64_t)blockIdx.x;
  // row block of residual slot i (split: one slot, block jb)
  auto mb_of = [&](int i) { return SPLIT ? jb : rh + 2 * i; };
  const float* xb = p.x + b * (int64_t)S * D;
  float* ob = p.out + b * (int64_t)S * D;

  // ---- residual stream: columns 32wc + 8q + 4g + e of row 32(rh + 2i) + rl ----
  f32x16 xr[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = mb_of(i) * 32 + rl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (m < S) v = *reinterpret_cast<const f32x4*>(xb + (int64_t)m * D + 32 * wc + 8 * q + 4 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) xr[i][4 * q + e] = v[e];
    }
  }

  // ---- weight fragments (A operand): W[n0 + rl][16*kk + 8g .. +8] ----
  // (wave-uniform base + 32-bit lane offset: the scalar-base addressing form)
  auto wfrag = [&](const f16* W, int K, int n0, int kk) {
    return *reinterpret_cast<const f16x8*>(W + (uint32_t)((n0 + rl) * K + 8 * g) + kk * 16);
  };
  // activation fragment (B operand): tile row r, k-step kk (+ chunk offset c0)
  auto afrag = [&](const char* T, int r, int c0, int kk) {
    return *reinterpret_cast<const f16x8*>(T + act_off(r, c0 + 2 * kk + g));
  };
  auto store_h4 = [&](char* T, int r, int n, const float (&v)[4]) {  // 4 consecutive n at n % 4 == 0
    const f16x4 t = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    *reinterpret_cast<f16x4*>(T + act_off(r, n >> 3) + (n & 7) * 2) = t;
  };

  // ---- LayerNorm of the residual stream (exact two passes over the 4 column waves) ----
  // FINAL: fp32 to the output; else fp16 into the h tile.
  auto layer_norm = [&](const float* gw, const float* gb, float eps, auto final_c) {
    constexpr bool FINAL = decltype(final_c)::value;
    refresh();
    float mean[2], rstd[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (SPLIT && i > 0) break;
      float s = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) s += xr[i][r];
      s = pair_sum(s);
      if (g == 0) stats[wc * kMaxRows + mb_of(i) * 32 + rl] = s;
    }
    lds_sync();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (SPLIT && i > 0) break;
      const int m = mb_of(i) * 32 + rl;
      mean[i] = (stats[m] + stats[kMaxRows + m] + stats[2 * kMaxRows + m] + stats[3 * kMaxRows + m]) / (float)D;
      float s = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float d = xr[i][r] - mean[i];
        s += d * d;
      }
      s = pair_sum(s);
      if (g == 0) stats[4 * kMaxRows + wc * kMaxRows + m] = s;
    }
    lds_sync();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (SPLIT && i > 0) break;
      const int m = mb_of(i) * 32 + rl;
      const float* s2 = stats + 4 * kMaxRows;
      const float var = (s2[m] + s2[kMaxRows + m] + s2[2 * kMaxRows + m] + s2[3 * kMaxRows + m]) / (float)D;
      rstd[i] = 1.0f / sqrtf(var + eps);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = 32 * wc + 8 * q + 4 * g;
      const f32x4 wv = *reinterpret_cast<const f32x4*>(gw + n);
      const f32x4 bv = *reinterpret_cast<const f32x4*>(gb + n);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (SPLIT && i > 0) break;
        const int m = mb_of(i) * 32 + rl;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (xr[i][4 * q + e] - mean[i]) * rstd[i] * wv[e] + bv[e];
        if constexpr (FINAL) {
          if (SPLIT && *lost) y[0] = y[1] = y[2] = y[3] = __builtin_nanf("");
          if (m < S) *reinterpret_cast<f32x4*>(ob + (int64_t)m * D + n) = f32x4{y[0], y[1], y[2], y[3]};
        } else {
          store_h4(Ht, m, n, y);
        }
      }
    }
  };

  // QKV weight blocks go through a two-deep buffer (block j in wq[j & 1]),
  // the others one phase ahead: at most two phases' fragments are live.
  f16x8 wq[2][KD], wo[KP], w1[KD], w2[KF];
  auto load_wq = [&](int l, int j) {
    const f16* W = p.w_qkv + (int64_t)l * 3 * DP * D;
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) wq[j & 1][kk] = wfrag(W, D, 32 * (wc + 4 * j), kk);
  };
  auto load_wo = [&](int l) {
#pragma unroll
    for (int kk = 0; kk < KP; ++kk) wo[kk] = wfrag(p.w_o + (int64_t)l * D * DP, DP, 32 * wc, kk);
  };
  auto load_w1 = [&](int l) {
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) w1[kk] = wfrag(p.w_1 + (int64_t)l * F * D, D, 32 * wc, kk);
  };
  auto load_w2 = [&](int l) {
#pragma unroll
    for (int kk = 0; kk < KF; ++kk) w2[kk] = wfrag(p.w_2 + (int64_t)l * D * F, F, 32 * wc, kk);
  };

  // V^T fragment offsets (see flash_dma_body): lane = 16*tq + ts covers
  // keys 16t + 8r + 4*(tq >> 1) + (ts >> 2), columns 32db + 16*(tq & 1) + 4*(ts & 3).
  const bool d_ok = HDP % 32 == 0 || (lane & 31) < HDP;
  const auto ones = __builtin_bit_cast(hf16x2, 0x3c003c00u);

  // layer l's vectors: thread t holds element t of each (b_qkv: elements t
  // and t + 256 with 256 threads), read from the arrays' layer-l rows.
  const int tid = threadIdx.x;
  const bool two_qkv = blockDim.x == 256;
  float vreg[9];
  auto vec_load = [&](int l) {
    if (tid < 3 * DP) vreg[0] = (p.b_qkv + l * 3 * DP)[(uint32_t)tid];
    if (two_qkv && tid + 256 < 3 * DP) vreg[8] = (p.b_qkv + l * 3 * DP)[(uint32_t)(tid + 256)];
    if (tid < D) {
      vreg[1] = (p.b_o + l * D)[(uint32_t)tid];
      vreg[2] = (p.b_1 + l * F)[(uint32_t)tid];
      vreg[3] = (p.b_2 + l * D)[(uint32_t)tid];
      vreg[4] = (p.n1_w + l * D)[(uint32_t)tid];
      vreg[5] = (p.n1_b + l * D)[(uint32_t)tid];
      vreg[6] = (p.n2_w + l * D)[(uint32_t)tid];
      vreg[7] = (p.n2_b + l * D)[(uint32_t)tid];
    }
  };
  auto vec_store = [&](int buf) {
    float* v = vecs + buf * VEC;
    if (tid < 3 * DP) v[tid] = vreg[0];
    if (two_qkv && tid + 256 < 3 * DP) v[tid + 256] = vreg[8];
    if (tid < D) {
      v[V_BO + tid] = vreg[1];
      v[V_B1 + tid] = vreg[2];
      v[V_B2 + tid] = vreg[3];
      v[V_N1W + tid] = vreg[4];
      v[V_N1B + tid] = vreg[5];
      v[V_N2W + tid] = vreg[6];
      v[V_N2B + tid] = vreg[7];
    }
  };
  // Split: K/V hand-off of layer l (after its QKV phase).  This block's K and V rows go to its
  // slot as they sit in its LDS tiles (the tiles' swizzle depends on the row only); once every
  // wave's stores have completed, its count of consumers (the later blocks) is published; an
  // earlier block's rows are read once its count is seen non-zero, and the count is decremented
  // when they are in LDS, so every count is back at 0 when the launch ends.
  // Ordering: the rows and the counts move only with agent-scope coherent accesses (sc1: what
  // the compiler emits for relaxed agent-scope atomics, each location coherent across the
  // device).  A producer's row stores have completed (vmcnt(0), every wave, then the barrier)
  // before its count is stored; a consumer issues its row loads after it has read the count.
  // So a consumer that sees the count reads the rows, without the release / acquire fences'
  // L2 write-back and invalidate (18 us of a 73 us C1 forward).
  auto exchange_kv = [&](int l) {
    const int64_t slot0 = ((int64_t)b * p.L + l) * 4;
    constexpr int kChunks = kSlotBytes / 16, kHalf = kChunks / 2;
    if (jb + 1 < MB) {
      char* dst = p.ws + (slot0 + jb) * kSlotBytes;
      for (int c = tid; c < kChunks; c += (int)blockDim.x) {
        const int half = c >= kHalf, off = (c - half * kHalf) * 16;
        const f32x4 v = *reinterpret_cast<const f32x4*>((half ? Vt : Kt) + jb * 32 * kPitch + off);
        asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(dst + half * (kSlotBytes / 2) + off), "v"(v)
                     : "memory");
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      if (tid == 0)
        __hip_atomic_store(p.flags + slot0 + jb, (unsigned)(MB - 1 - jb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (jb > 0) {
      if (tid < jb) {
        unsigned tries = 0;
        while (__hip_atomic_load(p.flags + slot0 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u &&
               ++tries < kSpinLimit)
          __builtin_amdgcn_s_sleep(2);
        if (tries >= kSpinLimit) *lost = 1;  // (its count is not decremented below)
      }
      __builtin_amdgcn_s_barrier();
      static_assert(kChunks == 4 * 256, "four 16-byte chunks per thread of a 256-thread workgroup");
      for (int blk = 0; blk < jb; ++blk) {
        const char* src = p.ws + (slot0 + blk) * kSlotBytes;
        const char* a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int c = tid + 256 * u, half = c >= kHalf;
          a[u] = src + half * (kSlotBytes / 2) + (c - half * kHalf) * 16;
        }
        // loads and their wait in one statement: the outputs are complete when it ends
        f32x4 v0, v1, v2, v3;
        asm volatile(
            "global_load_dwordx4 %0, %4, off sc1\n\t"
            "global_load_dwordx4 %1, %5, off sc1\n\t"
            "global_load_dwordx4 %2, %6, off sc1\n\t"
            "global_load_dwordx4 %3, %7, off sc1\n\t"
            "s_waitcnt vmcnt(0)"
            : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
            : "memory");
        const f32x4 vv[4] = {v0, v1, v2, v3};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int c = tid + 256 * u, half = c >= kHalf, off = (c - half * kHalf) * 16;
          *reinterpret_cast<f32x4*>((half ? Vt : Kt) + blk * 32 * kPitch + off) = vv[u];
        }
      }
      lds_sync();
      if (tid < jb && !*lost)
        __hip_atomic_fetch_add(p.flags + slot0 + tid, ~0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  vec_load(0);
  vec_store(0);
  if (threadIdx.x < D) {
    vecs[2 * VEC + threadIdx.x] = p.nf_w[threadIdx.x];
    vecs[2 * VEC + D + threadIdx.x] = p.nf_b[threadIdx.x];
  }
  if (threadIdx.x == 0) *lost = 0;
  load_wq(0, 0);
  lds_sync();  // vectors of layer 0 and the final norm staged
  layer_norm(vecs + V_N1W, vecs + V_N1B, p.n1_eps, std::false_type{});
  // Attention work items: (head, 32-row query block), heaviest first (causal
  // cost grows with the block index), dealt to the NWV waves in snake order.
  const int items = SPLIT ? p.H : p.H * MB;
  const int NWV = blockDim.x >> 6;
  for (int l = 0; l < p.L; ++l) {
    lds_sync();  // h complete
    // ---- QKV = h . W_qkv^T + b -> Q, K, V tiles ----
    {
      refresh();
      const float* bq = vecs + (l & 1) * VEC;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        if (j + 1 < NQ) load_wq(l, j + 1);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          if (SPLIT && i > 0) break;
          const int mb = mb_of(i);
          if (!SPLIT && mb >= MB) break;
          f32x16 acc = {};
#pragma unroll
          for (int kk = 0; kk < KD; ++kk)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(wq[j & 1][kk], afrag(Ht, mb * 32 + rl, 0, kk), acc, 0, 0, 0);
          const int nb = wc + 4 * j;  // 32-column block of [Q | K | V]
          const int part = nb / (DP / 32), col0 = (nb % (DP / 32)) * 32;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = 32 * nb + 8 * q + 4 * g;
            const f32x4 bv = *reinterpret_cast<const f32x4*>(bq + n);
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[4 * q + e] + bv[e];
            const int c = col0 + 8 * q + 4 * g, r = mb * 32 + rl;
            if (part == 2) {
              const f16x4 t = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
              *reinterpret_cast<f16x4*>(Vt + v_off(r, c >> 3) + (c & 7) * 2) = t;
            } else {
              store_h4(part == 0 ? Qt : Kt, r, c, v);
            }
          }
        }
      }
    }
    // W_o's fragments load under the attention phase; at head_dim 128 its
    // 64-register O leaves no room for them, so they follow it.
    if constexpr (HDP < 128) load_wo(l);
    if (l + 1 < p.L) vec_load(l + 1);
    lds_sync();  // Q, K, V complete
    if constexpr (SPLIT) exchange_kv(l);
    // ---- attention over this wave's (head, query block) items; ctx -> h tile ----
    for (int k = 0; k < items; ++k) {
      refresh();
      const int kr = k % (2 * NWV);
      if ((kr < NWV ? kr : 2 * NWV - 1 - kr) != w) continue;
      const int qb = SPLIT ? jb : MB - 1 - k / p.H;
      const int hh = k % p.H;
      const int hc = hh * HDP / 8;  // first chunk of this head's columns
      const int row = qb * 32 + rl;
      // Q^T fragments: held in registers for the item, or at head_dim 128
      // (32 registers beside a 64-register O) re-read from LDS per key block.
      constexpr bool Q_REG = HK < 8;
      f16x8 qf[Q_REG ? HK : 1];
      if constexpr (Q_REG) {
#pragma unroll
        for (int kk = 0; kk < HK; ++kk) qf[kk] = afrag(Qt, row, hc, kk);
      }
      const int kb_end = CAUSAL ? qb + 1 : MB;
      // Online softmax over the 32-key blocks (S^T = K . Q^T: a lane holds 16
      // keys of query `row`, its partner lane the other 16): running max m_run
      // (in exp2 units), O and the row sum rescaled when it grows.  Key block
      // 0 holds a valid key for every row, so m_run is finite from there on.
      const float cs = p.scale_log2;
      float m_run = -INFINITY, ls = 0.f;
      f32x16 oacc[DB];
#pragma unroll
      for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        if (kb < kb_end) {
          f32x16 a = {};
#pragma unroll
          for (int kk = 0; kk < HK; ++kk)
            a = __builtin_amdgcn_mfma_f32_32x32x16_f16(afrag(Kt, kb * 32 + rl, hc, kk),
                                                       Q_REG ? qf[Q_REG ? kk : 0] : afrag(Qt, row, hc, kk), a, 0, 0, 0);
          float mx = -INFINITY;
          if ((CAUSAL && kb == qb) || kb * 32 + 32 > S) {  // the diagonal block, the block holding key S-1
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
              if (key >= S || (CAUSAL && key > row)) a[r] = -INFINITY;
              mx = fmaxf(mx, a[r]);
            }
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, a[r]);
          }
          const float m_new = fmaxf(m_run, pair_max(mx) * cs);  // cs > 0: max(s)*cs == max(s*cs)
          if (kb > 0) {
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            ls *= alpha;
#pragma unroll
            for (int d = 0; d < DB; ++d)
#pragma unroll
              for (int r = 0; r < 16; ++r) oacc[d][r] *= alpha;
          }
          m_run = m_new;
          f16x8 pf[2];
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            const f16x2 hp = {(f16)__builtin_amdgcn_exp2f(fmaf(a[e], cs, -m_new)),
                              (f16)__builtin_amdgcn_exp2f(fmaf(a[e + 1], cs, -m_new))};
            pf[e >> 3][e & 7] = hp[0];
            pf[e >> 3][(e & 7) + 1] = hp[1];
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(hf16x2, hp), ones, ls, false);
          }
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const int t = 2 * kb + tt;
#pragma unroll
            for (int d = 0; d < DB; ++d) {
              f16x4 half[2];
#pragma unroll
              for (int r = 0; r < 2; ++r) {
                const int vr = 16 * t + 8 * r + 4 * (tq >> 1) + (ts >> 2);
                const int col = hh * HDP + 32 * d + (HDP >= 32 ? 16 * (tq & 1) : 0) + 4 * (ts & 3);
                const tr_f16x4 x4 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (lds_tr_f16x4*)(lds_char*)(Vt + v_off(vr, col >> 3) + (col & 7) * 2));
                half[r] = __builtin_bit_cast(f16x4, x4);
              }
              f16x8 vf = __builtin_shufflevector(half[0], half[1], 0, 1, 2, 3, 4, 5, 6, 7);
              if (!d_ok) vf = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
              oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[tt], oacc[d], 0, 0, 0);
            }
          }
        }
      }
      const float inv = 1.0f / pair_sum(ls);
      // lane holds O[row][32d + 8q + 4g + e]
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int dd = 32 * d + 8 * q + 4 * g;
          if (dd < HDP) {
            const float v[4] = {oacc[d][4 * q] * inv, oacc[d][4 * q + 1] * inv, oacc[d][4 * q + 2] * inv,
                                oacc[d][4 * q + 3] * inv};
            store_h4(Ht, row, hh * HDP + dd, v);
          }
        }
    }
    if constexpr (HDP == 128) load_wo(l);
    load_w1(l);
    lds_sync();  // ctx complete
    // ---- x += ctx . W_o^T + b_o ----
    {
      refresh();
      const f32x4* bo4 = reinterpret_cast<const f32x4*>(vecs + (l & 1) * VEC + V_BO + 32 * wc + 4 * g);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (SPLIT && i > 0) break;
        const int mb = mb_of(i);
        if (!SPLIT && mb >= MB) break;
        f32x16 acc = {};
#pragma unroll
        for (int kk = 0; kk < KP; ++kk)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(wo[kk], afrag(Ht, mb * 32 + rl, 0, kk), acc, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 bv = bo4[2 * q];
#pragma unroll
          for (int e = 0; e < 4; ++e) xr[i][4 * q + e] = xr[i][4 * q + e] + (acc[4 * q + e] + bv[e]);
        }
      }
    }
    load_w2(l);
    layer_norm(vecs + (l & 1) * VEC + V_N2W, vecs + (l & 1) * VEC + V_N2B, p.n2_eps, std::false_type{});
    lds_sync();  // h complete
    // ---- u = gelu(h . W_1^T + b_1) -> u tile (reuses Q) ----
    {
      refresh();
      const f32x4* b14 = reinterpret_cast<const f32x4*>(vecs + (l & 1) * VEC + V_B1 + 32 * wc + 4 * g);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (SPLIT && i > 0) break;
        const int mb = mb_of(i);
        if (!SPLIT && mb >= MB) break;
        f32x16 acc = {};
#pragma unroll
        for (int kk = 0; kk < KD; ++kk)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(w1[kk], afrag(Ht, mb * 32 + rl, 0, kk), acc, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 bv = b14[2 * q];
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = gelu_erf(acc[4 * q + e] + bv[e]);
          store_h4(Qt, mb * 32 + rl, 32 * wc + 8 * q + 4 * g, v);
        }
      }
    }
    if (l + 1 < p.L) vec_store((l + 1) & 1);  // layer l+1's vectors (its LN1 runs below)
    lds_sync();  // u complete
    if (l + 1 < p.L) load_wq(l + 1, 0);
    // ---- x += u . W_2^T + b_2 ----
    {
      refresh();
      const f32x4* b24 = reinterpret_cast<const f32x4*>(vecs + (l & 1) * VEC + V_B2 + 32 * wc + 4 * g);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (SPLIT && i > 0) break;
        const int mb = mb_of(i);
        if (!SPLIT && mb >= MB) break;
        f32x16 acc = {};
#pragma unroll
        for (int kk = 0; kk < KF; ++kk)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(w2[kk], afrag(Qt, mb * 32 + rl, 0, kk), acc, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 bv = b24[2 * q];
#pragma unroll
          for (int e = 0; e < 4; ++e) xr[i][4 * q + e] = xr[i][4 * q + e] + (acc[4 * q + e] + bv[e]);
        }
      }
    }
    if (l + 1 < p.L)
      layer_norm(vecs + ((l + 1) & 1) * VEC + V_N1W, vecs + ((l + 1) & 1) * VEC + V_N1B, p.n1_eps,
                 std::false_type{});
    else
      layer_norm(vecs + 2 * VEC, vecs + 2 * VEC + D, p.nf_eps, std::true_type{});
  }
}

template <int HDP, bool CAUSAL>
int launch_small(const SmallArgs& p, int64_t batch, hipStream_t st) {
  if constexpr (CAUSAL) {
    if (p.ws != nullptr) {  // split: one 32-row block per workgroup, 4 waves
      const unsigned blocks = (unsigned)batch * (unsigned)((p.S + 31) / 32);
      hipLaunchKernelGGL((small_forward_kernel<128, 128, 128, HDP, true, true>), dim3(blocks), dim3(256), 0, st, p);
      return check_launch("tk_small_forward");
    }
  }
  // 8 waves: column block w & 3, row blocks (w >> 2) + {0, 2}.  A single row
  // block (S <= 32) leaves waves 4-7 without rows: 4 waves then.
  const unsigned threads = p.S <= 32 ? 256 : 512;
  hipLaunchKernelGGL((small_forward_kernel<128, 128, 128, HDP, CAUSAL, false>), dim3((unsigned)batch), dim3(threads),
                     0, st, p);
  return check_launch("tk_small_forward");
}

// Compute units of the current device (cached per device).
int device_cus(int dev) {
  static int cus[64] = {0};
  if (dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 1;
    cus[dev] = n;
  }
  return cus[dev];
}

// The split launch's hand-off workspace: a table of kMaxSlots consumer counts at a fixed place
// (its start), then 4 block slots of K and V rows per (sequence, layer) -- count i belongs to
// slot i.  Every launch leaves the counts it used at 0 and slots never overlap the table, so the
// counts are 0 at every launch's start whatever shapes the workspace served before.
constexpr int64_t kMaxSlots = 4096;                  // batch x layers x 4 (C1: 1024)
constexpr int64_t kCountBytes = kMaxSlots * 4;
int64_t split_ws_bytes(int64_t batch, int64_t layers) { return kCountBytes + batch * layers * 4 * kSlotBytes; }

// Whether a shape runs split (one 32-row block per workgroup): causal, more than one row block,
// every workgroup resident at once (batch x blocks <= CUs; a waiting block's producers then run).
bool use_split(int64_t batch, int64_t seq, int64_t layers, bool causal, int dev) {
  const int64_t mb = (seq + 31) / 32;
  return causal && mb > 1 && batch * mb <= device_cus(dev) && batch * layers * 4 <= kMaxSlots;
}

// The split launch's workspace: one zeroed buffer per device, replaced by one at least twice as
// large when a call needs more; kernels leave every consumer count at 0.  An outgrown buffer is
// kept, not freed (a captured graph may still launch with it), so the device holds at most about
// twice the largest workspace.  Never allocated while the stream is being captured (the call then
// runs unsplit).
std::mutex g_ws_mutex;
struct Workspace {
  char* ptr = nullptr;
  int64_t bytes = 0;
};
Workspace g_ws[64];

char* split_workspace(int dev, int64_t bytes, hipStream_t st) {
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace& w = g_ws[dev];
  if (w.bytes >= bytes) return w.ptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  const int64_t want = std::max(bytes, 2 * w.bytes);
  char* ptr = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&ptr), (size_t)want) != hipSuccess) return nullptr;
  if (hipMemsetAsync(ptr, 0, (size_t)want, st) != hipSuccess) {
    (void)hipFree(ptr);
    return nullptr;
  }
  w.ptr = ptr;
  w.bytes = want;
  return ptr;
}

}  // namespace
}  // namespace tk

using namespace tk;

extern "C" int tk_small_forward_supported(int64_t seq, int64_t d_model, int64_t heads, int64_t head_dim_padded,
                                          int64_t ffn_dim) {
  const int64_t hp = head_dim_padded;
  return seq >= 1 && seq <= kMaxRows && d_model == 128 && ffn_dim == 128 && heads >= 1 &&
         (hp == 16 || hp == 32 || hp == 64 || hp == 128) && heads * hp == 128;
}

// Scratch of tk_small_forward_noalloc (the split launch's count table and hand-off slots): a
// fixed array of every device, located per device once with hipGetSymbolAddress.
constexpr int64_t kNoAllocSlots = 1024;  // batch x layers x 4 blocks (C1: 1024)
static __device__ __attribute__((aligned(256))) char scratch[kCountBytes + kNoAllocSlots * kSlotBytes];

namespace {

std::mutex g_scratch_mutex;
char* g_scratch[64];

// Device address of this device's scratch (the device current), or nullptr.
char* scratch_address(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return nullptr;
    g_scratch[dev] = static_cast<char*>(ptr);
  }
  return g_scratch[dev];
}

__global__ void clear_counts(unsigned* counts, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) counts[i] = 0u;
}

int small_forward_call(const char* fn, bool noalloc, const float* x, float* out, int64_t batch, int64_t seq,
                       int64_t d_model, int64_t heads, int64_t head_dim_padded, int64_t ffn_dim, int64_t layers,
                       int causal, const tk_half* w_qkv, const float* b_qkv, const tk_half* w_o, const float* b_o,
                       const tk_half* w_1, const float* b_1, const tk_half* w_2, const float* b_2, const float* n1_w,
                       const float* n1_b, const float* n2_w, const float* n2_b, const float* nf_w,
                       const float* nf_b, float n1_eps, float n2_eps, float nf_eps, float scale, void* stream) {
  clear_error();
  TK_REQUIRE(x && out && w_qkv && b_qkv && w_o && b_o && w_1 && b_1 && w_2 && b_2 && n1_w && n1_b && n2_w &&
                 n2_b && nf_w && nf_b,
             TK_ERR_ARG, "%s: null pointer", fn);
  TK_REQUIRE(tk_small_forward_supported(seq, d_model, heads, head_dim_padded, ffn_dim), TK_ERR_UNSUPPORTED,
             "%s: shape S=%lld D=%lld H=%lld hd=%lld F=%lld outside the kernel's "
             "(S <= 128, D = F = 128, H*hd = 128, hd in {16,32,64,128})",
             fn, (long long)seq, (long long)d_model, (long long)heads, (long long)head_dim_padded,
             (long long)ffn_dim);
  TK_REQUIRE(batch >= 0 && batch < (1ll << 31) && layers >= 1 && layers < (1 << 20), TK_ERR_ARG,
             "%s: batch=%lld layers=%lld", fn, (long long)batch, (long long)layers);
  TK_REQUIRE(scale > 0.f, TK_ERR_ARG, "%s: scale must be > 0", fn);
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  TK_REQUIRE(al16(x) && al16(out) && al16(w_qkv) && al16(w_o) && al16(w_1) && al16(w_2) && al16(b_qkv) &&
                 al16(b_o) && al16(b_1) && al16(b_2) && al16(n1_w) && al16(n1_b) && al16(n2_w) && al16(n2_b) &&
                 al16(nf_w) && al16(nf_b),
             TK_ERR_ARG, "%s: every buffer must be 16-byte aligned", fn);
  if (batch == 0) return TK_OK;
  SmallArgs p;
  p.x = x;
  p.out = out;
  p.w_qkv = reinterpret_cast<const f16*>(w_qkv);
  p.b_qkv = b_qkv;
  p.w_o = reinterpret_cast<const f16*>(w_o);
  p.b_o = b_o;
  p.w_1 = reinterpret_cast<const f16*>(w_1);
  p.b_1 = b_1;
  p.w_2 = reinterpret_cast<const f16*>(w_2);
  p.b_2 = b_2;
  p.n1_w = n1_w;
  p.n1_b = n1_b;
  p.n2_w = n2_w;
  p.n2_b = n2_b;
  p.nf_w = nf_w;
  p.nf_b = nf_b;
  p.n1_eps = n1_eps;
  p.n2_eps = n2_eps;
  p.nf_eps = nf_eps;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.S = (int)seq;
  p.L = (int)layers;
  p.H = (int)heads;
  hipStream_t st = as_stream(stream);
  const bool c = causal != 0;
  p.B = (int)batch;
  p.ws = nullptr;
  p.flags = nullptr;
  int dev = 0;
  TK_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64, TK_ERR_HIP, "%s: no device", fn);
  if (use_split(batch, seq, layers, c, dev)) {
    if (noalloc) {
      // the device's static scratch: its count table is cleared first (a previous call on this
      // device leaves it at 0 unless that call failed)
      const int64_t slots = batch * layers * 4;
      TK_REQUIRE(slots <= kNoAllocSlots, TK_ERR_UNSUPPORTED,
                 "%s: batch %lld x layers %lld x 4 row blocks = %lld hand-off slots, more than the %lld of the "
                 "static scratch (16 MB); use tk_small_forward",
                 fn, (long long)batch, (long long)layers, (long long)slots, (long long)kNoAllocSlots);
      char* ws = scratch_address(dev);
      TK_REQUIRE(ws != nullptr, TK_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed", fn);
      hipLaunchKernelGGL(clear_counts, dim3((unsigned)(kMaxSlots / 256)), dim3(256), 0, st,
                         reinterpret_cast<unsigned*>(ws), (int)kMaxSlots);
      p.flags = reinterpret_cast<unsigned*>(ws);
      p.ws = ws + kCountBytes;
    } else {
      char* ws = split_workspace(dev, split_ws_bytes(batch, layers), st);
      if (ws != nullptr) {
        p.flags = reinterpret_cast<unsigned*>(ws);
        p.ws = ws + kCountBytes;
      }
    }
  }
  switch (head_dim_padded) {
    case 16: return c ? launch_small<16, true>(p, batch, st) : launch_small<16, false>(p, batch, st);
    case 32: return c ? launch_small<32, true>(p, batch, st) : launch_small<32, false>(p, batch, st);
    case 64: return c ? launch_small<64, true>(p, batch, st) : launch_small<64, false>(p, batch, st);
    default: return c ? launch_small<128, true>(p, batch, st) : launch_small<128, false>(p, batch, st);
  }
}

}  // namespace

extern "C" int tk_small_forward(const float* x, float* out, int64_t batch, int64_t seq, int64_t d_model,
                                int64_t heads, int64_t head_dim_padded, int64_t ffn_dim, int64_t layers, int causal,
                                const tk_half* w_qkv, const float* b_qkv, const tk_half* w_o, const float* b_o,
                                const tk_half* w_1, const float* b_1, const tk_half* w_2, const float* b_2,
                                const float* n1_w, const float* n1_b, const float* n2_w, const float* n2_b,
                                const float* nf_w, const float* nf_b, float n1_eps, float n2_eps, float nf_eps,
                                float scale, void* stream) {
  return small_forward_call("tk_small_forward", false, x, out, batch, seq, d_model, heads, head_dim_padded, ffn_dim,
                            layers, causal, w_qkv, b_qkv, w_o, b_o, w_1, b_1, w_2, b_2, n1_w, n1_b, n2_w, n2_b, nf_w,
                            nf_b, n1_eps, n2_eps, nf_eps, scale, stream);
}

extern "C" int tk_small_forward_noalloc(const float* x, float* out, int64_t batch, int64_t seq, int64_t d_model,
                                        int64_t heads, int64_t head_dim_padded, int64_t ffn_dim, int64_t layers,
                                        int causal, const tk_half* w_qkv, const float* b_qkv, const tk_half* w_o,
                                        const float* b_o, const tk_half* w_1, const float* b_1, const tk_half* w_2,
                                        const float* b_2, const float* n1_w, const float* n1_b, const float* n2_w,
                                        const float* n2_b, const float* nf_w, const float* nf_b, float n1_eps,
                                        float n2_eps, float nf_eps, float scale, void* stream) {
  return small_forward_call("tk_small_forward_noalloc", true, x, out, batch, seq, d_model, heads, head_dim_padded,
                            ffn_dim, layers, causal, w_qkv, b_qkv, w_o, b_o, w_1, b_1, w_2, b_2, n1_w, n1_b, n2_w,
                            n2_b, nf_w, nf_b, n1_eps, n2_eps, nf_eps, scale, stream);
}
