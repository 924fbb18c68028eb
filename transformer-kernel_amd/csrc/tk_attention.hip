// FlashAttention-2-style forward for gfx950 (fp16 MFMA, fp32 online softmax).
//
// Per workgroup: BM = 32*NW query rows of one (batch, head), one wave per 32
// rows, key/value tiles of 64 keys in LDS.
//
// Transposed formulation (both kernel bodies).  Each wave computes
// S^T = K . Q^T with v_mfma_f32_32x32x16_f16 (A operand = K rows from LDS,
// B operand = the wave's Q rows, held in registers for the whole kernel).
// In the 32x32 accumulator layout a lane then holds 16 keys of ONE query row
// (row = lane & 31; lanes l and l^32 hold the two halves), so
//   * the running max / sum of a row need one lane-pair exchange, no LDS;
//   * the rescale of the output accumulator is one scalar per lane;
//   * the fp16 probabilities of 8 consecutive accumulator entries are
//     directly the B operand of O^T = V^T . P^T; those 8 entries stand for
//     the keys {16t + 8*e2 + 4g + e10} (g = lane >> 5).
//
// Two bodies, picked by head_dim at compile time:
//   flash_dma_body (head_dim <= 64): K and V tiles copied global -> LDS
//     directly (global_load_lds_dwordx4, row-major); the V^T operand is two
//     ds_read_b64_tr_b16 of the row-major V tile.  The O^T MFMAs of tile t-1
//     are deferred into step t, so every MFMA of a step is independent of
//     the step's exponentials and interleaves with them; the row max of the
//     next tile is computed in the same pass.
//   flash_vreg_body (head_dim 128): the deferred P needs 16 more registers
//     than two waves per SIMD leave at head_dim 128, so tile t's O^T MFMAs
//     follow its exponentials; V^T is written to LDS from registers with
//     key bits 2 and 3 swapped so that each A operand is one 16-byte read.
//   Measured on MI355X (C5 shape, head_dim 64): the DMA body 5.6-5.8 ms
//   against 6.2-6.3 ms for the register body; at head_dim 128 (C4 shape)
//   the register body 1.48 ms against 1.70 ms.
//
// Numerics (src/kernels.py:112-134, src/torch_transformer_benchmark.py:97-111):
// fp32 scores, the scale applied in fp32 after Q.K^T (folded with log2(e)
// into one FMA before exp2: exp2(s*c - m*c) = exp(scale*(s - m))), -inf
// masking of future and invalid keys, fp32 running max and sums, fp16 P for
// the PV product, fp32 accumulation, one final divide.
#include "tk_attn_tile.hpp"

namespace tk {
namespace {

constexpr int kBN = 64;     // keys per tile
constexpr int kKSlots = 2;  // flash_dma_body K tiles in LDS: t+1 (read), t+2 (landing)


// s_waitcnt vmcnt(0) with the other counters unconstrained (gfx9 encoding).
__device__ __forceinline__ void wait_copies() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }

template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

struct AttnArgs {
  const f16* q;
  const f16* k;
  const f16* v;
  f16* o;
  int64_t qs[3], ks[3], vs[3], os[3];  // element strides for (b, h, s)
  const uint8_t* kv;                   // nullable key validity, [b * kvs + key]
  int64_t kvs;
  int B, H, S;
  float scale_log2;  // scale * log2(e)
};

// ---- register-staged V (flash_vreg_body) ----
constexpr int kStages = 3;  // LDS stages (tile t read, t+1 read as "next K", t+2 landing)

typedef __attribute__((address_space(3))) void lds_void;

// Position of key k (0..63 within the tile) in a V^T row: bits 2 and 3 swapped.
__device__ __forceinline__ int vpos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

// The bodies are __device__ functions (the __global__ wrapper below only
// calls them): device-only builtins used directly in a kernel template's
// lambdas would make the host-side instantiation, and with it the launch
// stub, fail.  KMASK: the key-validity mask p.kv is applied (a separate
// instantiation, so the unmasked kernels carry none of its registers or
// loads).
template <int HD, int NW, bool CAUSAL, bool KMASK>
__device__ __forceinline__ void flash_dma_body(const AttnArgs& p) {
  constexpr int BM = 32 * NW;
  constexpr int RB = HD * 2;               // K / V tile row bytes
  constexpr int CPR = RB / 16;             // 16-byte chunks per row
  constexpr int TILE = kBN * RB;           // bytes per K or V tile
  constexpr int COPIES = TILE / 1024;      // 1 KB wave copies per tile
  constexpr int CPW = (COPIES + NW - 1) / NW;
  constexpr int RPC = 1024 / RB;           // tile rows per copy
  constexpr int DB = (HD + 31) / 32;       // 32-row blocks of the O^T accumulator
  constexpr int KSTEPS = HD / 16;          // k16 steps of S^T = K.Q^T
  constexpr int NS = 2 * KSTEPS;           // S^T MFMAs per tile
  constexpr int NP = 4 * DB;               // O^T MFMAs per tile
  // The O^T MFMAs of tile t-1 are deferred into step t (V tiles t-1, t, t+1
  // in LDS).
  constexpr int kVSlots = 3;
  constexpr int NM = NS + NP;  // MFMAs of the interleaved chunk region
  constexpr int NC = NM / 2 < 4 ? 4 : NM / 2;  // chunks per step
  constexpr int EPC = 32 / NC;             // score entries per lane per chunk
  static_assert(HD <= 64, "head_dim 128 takes the ring / pair / register bodies, 256 the generic kernel");
  static_assert(TILE % 1024 == 0, "tiles must be whole 1 KB copies");
  static_assert(32 % NC == 0 && EPC % 2 == 0, "chunks must split the 32 entries into pairs");

  __shared__ __attribute__((aligned(16))) char smem[(kKSlots + kVSlots) * TILE];
  const uint32_t lds_base = (uint32_t)(size_t)(lds_char*)smem;
  auto kslot = [&](int i) { return smem + i * TILE; };
  auto vslot = [&](int i) { return smem + (kKSlots + i) * TILE; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const uint8_t* kvb = KMASK ? p.kv + b * p.kvs : nullptr;

  const int my_row = q0 + wave * 32 + (lane & 31);
  const int g = lane >> 5;
  const int wave_row_min = q0 + wave * 32;

  // Q^T fragments (B operand): lane supplies Q[row][16*kk + 8*g .. +8].
  f16x8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    if (my_row < p.S)
      qf[kk] = *reinterpret_cast<const f16x8*>(qb + (int64_t)my_row * p.qs[2] + kk * 16 + g * 8);
    else
      qf[kk] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  wait_copies();  // Q is in registers before any copy is issued

  f32x16 acc_o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[d][r] = 0.f;
  float m_run = -INFINITY;  // running max of scale*log2e*s
  float l_run = 0.f;        // lane-partial running sum (this lane's keys)

  const int kv_end = CAUSAL ? min(p.S, q0 + BM) : p.S;
  const int n_kt = (kv_end + kBN - 1) / kBN;

  // ---- copies: lane sources within a tile are fixed; a tile adds 64 rows ----
  // Lane l of wave copy ci writes physical chunk l % CPR of tile row
  // ci*RPC + l / CPR and fetches the logical chunk the swizzle maps there.
  int c_row[CPW], k_col[CPW], v_col[CPW];
  const f16* k_src[CPW];
  const f16* v_src[CPW];
  auto copy_setup = [&](int ln) {
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int ci = wave + i * NW;
      const int row = ci * RPC + ln / CPR;
      const int phys = ln % CPR;
      c_row[i] = row;
      k_col[i] = ((swz_off<RB>(row, phys) - row * RB) >> 4) * 8;  // the XOR is an involution
      v_col[i] = (phys ^ vswz<RB>(row)) * 8;
      k_src[i] = kb + (int64_t)row * p.ks[2] + k_col[i];
      v_src[i] = vb + (int64_t)row * p.vs[2] + v_col[i];
    }
  };
  copy_setup(lane);
  const int64_t k_tile = (int64_t)kBN * p.ks[2], v_tile = (int64_t)kBN * p.vs[2];
  auto copy_tile = [&](const f16* const (&src)[CPW], const f16* base, int64_t rs, int64_t tstride,
                       const int (&col)[CPW], int j, uint32_t dst) {
    if ((j + 1) * kBN <= p.S) {
#pragma unroll
      for (int i = 0; i < CPW; ++i)
        if (COPIES % NW == 0 || wave + i * NW < COPIES)
          dma16(src[i] + j * tstride, dst + (wave + i * NW) * 1024);
    } else {  // last tile: rows past S re-read row S-1 (finite; masked or multiplied by P = 0)
#pragma unroll
      for (int i = 0; i < CPW; ++i)
        if (COPIES % NW == 0 || wave + i * NW < COPIES) {
          const int key = min(j * kBN + c_row[i], p.S - 1);
          dma16(base + (int64_t)key * rs + col[i], dst + (wave + i * NW) * 1024);
        }
    }
  };
  auto copy_k = [&](int j) { copy_tile(k_src, kb, p.ks[2], k_tile, k_col, j, lds_base + (j % kKSlots) * TILE); };
  auto copy_v = [&](int j) {
    copy_tile(v_src, vb, p.vs[2], v_tile, v_col, j, lds_base + (kKSlots + j % kVSlots) * TILE);
  };

  // ---- operand reads ----
  // A operand of S^T MFMA c (key block c / KSTEPS, k-step c % KSTEPS).
  auto read_k = [&](const char* ks_, int c) {
    return *reinterpret_cast<const f16x8*>(ks_ + swz_off<RB>((c / KSTEPS) * 32 + (lane & 31), 2 * (c % KSTEPS) + g));
  };
  // A operand of O^T MFMA c: P column block t = c / DB, head-dim block c % DB.
  // lane = 16*q + s; read r (0/1) covers keys 16t + 8r + 4*(q >> 1) + (s >> 2)
  // and head-dim columns 32*db + 16*(q & 1) + 4*(s & 3); the swizzle only sees
  // row bits 0-1, which 16t leaves unchanged.
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
  const bool d_ok = HD % 32 == 0 || (lane & 31) < HD;  // head-dim row of this lane's O^T entries exists
  auto read_v = [&](const char* vs_, int c) -> f16x8 {
    const int t = c / DB, d = c % DB;
    const lds_char* base = (const lds_char*)(vs_ + t * 16 * RB);
    const tr_f16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[0][d]));
    const tr_f16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[1][d]));
    const f16x8 f = __builtin_shufflevector(__builtin_bit_cast(f16x4, lo), __builtin_bit_cast(f16x4, hi), 0, 1, 2,
                                            3, 4, 5, 6, 7);
    return d_ok ? f : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  };
  // O^T += V^T . P^T for a whole tile (the last tile).
  auto pv_all = [&](const f16x8 (&pf)[4], const char* vs_) {
#pragma unroll
    for (int c = 0; c < NP; ++c)
      acc_o[c % DB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_v(vs_, c), pf[c / DB], acc_o[c % DB], 0, 0, 0);
  };

  // Key validity of a tile as one 64-bit ballot (bit j: key k0 + j valid).
  // The byte of tile kt+1 is loaded at the start of step kt and turned into
  // bits after the step's copy wait, so no wait for it lands mid-step.
  auto key_byte = [&](int kt) { return KMASK ? (int)kvb[min(kt * kBN + lane, p.S - 1)] : 1; };
  uint64_t kbits_cur = KMASK ? (uint64_t)__ballot(key_byte(0) != 0) : 0ull;
  const auto ones = __builtin_bit_cast(hf16x2, 0x3c003c00u);

  // One tile step kt (see the header).  accumulator entry r of block kb2 is
  // key k0 + 32*kb2 + 8*(r/4) + 4*g + r%4.
  auto step = [&](int kt, f32x16 (&s_cur)[2], f32x16 (&s_next)[2], f16x8 (&p_cur)[4], f16x8 (&p_prev)[4],
                  float& mx_cur, float& mx_next, auto next_c, auto prev_c) {
    constexpr bool HAS_NEXT = decltype(next_c)::value;
    constexpr bool HAS_PREV = decltype(prev_c)::value;
    const int k0 = kt * kBN;
    // The copies go out from inside the chunk loop (K after chunk 0, V after
    // chunk 2) rather than here: issued right after the barrier, every wave
    // of the CU queues its copies at once and stalls on issue before its
    // first MFMA.  Their LDS slots (tile kt's K, tile kt-2's V) are free
    // since the previous step's barrier.
    constexpr int C_K = 0, C_V = NC > 2 ? 2 : NC - 1;
    int kbyte_next = 1;
    if (KMASK && HAS_NEXT) kbyte_next = key_byte(kt + 1);

    const bool need_mask = (k0 + kBN > p.S) || (CAUSAL && k0 + kBN - 1 > wave_row_min) || KMASK;
    // Steps after the first on unmasked tiles (m_run finite) rescale only when needed: P(kt)
    // is computed against m_run and, when its row sum reaches 65504 (the fp16 maximum, so
    // before any entry could overflow fp16; or NaN), the tile's max moves m_run and P(kt) is
    // computed again (after the slots below).
    const bool fit_test = !KMASK && !need_mask && kt > 0;
    float mx = mx_cur;
    if (need_mask) {
      // bit j of kbits: key k0 + 4*g + j is valid
      const uint64_t kbits = kbits_cur >> (4 * g);
      mx = -INFINITY;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = kb2 * 32 + 8 * (r >> 2) + (r & 3);
          const int key = k0 + j + 4 * g;
          if (key >= p.S || (CAUSAL && key > my_row) || (KMASK && ((kbits >> j) & 1) == 0))
            s_cur[kb2][r] = -INFINITY;
          mx = fmaxf(mx, s_cur[kb2][r]);
        }
    }
    const float cs = p.scale_log2;
    // Lazy rescale (the other steps): the reference max m_run only moves when
    // some row of the wave has grown by more than 2^8 over it, so exponentials
    // stay <= 256 and the O/l rescale is skipped on most tiles; O and l always
    // share one reference, so the final O/l is unchanged.  l (tiles < kt) is
    // rescaled here.  With deferred P.V, O is rescaled at the end of the step,
    // after the deferred MFMAs have added tile kt-1 at the old reference, so no
    // MFMA writes O on a conditional path (an MFMA accumulator written on two
    // paths is copied between register sets on every step).
    mx = pair_max(mx);
    const float m_tile = mx * cs;  // cs > 0: max(s)*cs == max(s*cs)
    bool rescale = !fit_test && __any(m_tile > m_run + 8.0f);
    float alpha = 1.0f;
    if (rescale) {
      const float m_new = fmaxf(m_run, m_tile);
      alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
    }
    float m_use = m_run == -INFINITY ? 0.f : m_run;

    // ---- chunks: MFMAs m in [c*NM/NC, (c+1)*NM/NC): S^T(kt+1) first, then O^T(kt-1) ----
    const char* ks_n = kslot((kt + 1) % kKSlots);
    const char* vs_p = vslot((kt + kVSlots - 1) % kVSlots);
    f16x8 frag[NM];
    auto issue_read = [&](int m) {
      if (m < NS) {
        if (HAS_NEXT) frag[m] = read_k(ks_n, m);
      } else if (m < NM) {
        if (HAS_PREV) frag[m] = read_v(vs_p, m - NS);
      }
    };
    auto do_mfma = [&](int m) {
      if (m < NS) {
        if (HAS_NEXT) {
          const int kb2 = m / KSTEPS, kk = m % KSTEPS;
          s_next[kb2] =
              __builtin_amdgcn_mfma_f32_32x32x16_f16(frag[m], qf[kk], kk == 0 ? f32x16{} : s_next[kb2], 0, 0, 0);
        }
      } else if (HAS_PREV) {
        const int c = m - NS;
        acc_o[c % DB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag[m], p_prev[c / DB], acc_o[c % DB], 0, 0, 0);
      }
    };
    float pe[32];
    float ls = 0.f;
    auto exp_entry = [&](int e) {
      pe[e] = __builtin_amdgcn_exp2f(fmaf(s_cur[e >> 4][e & 15], cs, -m_use));
      if (e & 1) {
        const f16x2 hp = {(f16)pe[e - 1], (f16)pe[e]};
        p_cur[e >> 3][(e & 7) - 1] = hp[0];
        p_cur[e >> 3][e & 7] = hp[1];
        // Row sum.  Causal: the fp32 exponentials in entry order, as the asm loop (two
        // adds per pair cost less beside the MFMAs than one fp16 dot of the packed pair);
        // non-causal (no asm loop): the fp16 dot, which keeps these instantiations within
        // 256 VGPRs without scratch.
        if constexpr (CAUSAL) {
          ls += pe[e - 1];
          ls += pe[e];
        } else {
          ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(hf16x2, hp), ones, ls, false);
        }
      }
    };
    // Reads run three MFMAs ahead of their use.
    constexpr int RA = 3;
#pragma unroll
    for (int m = 0; m < RA && m < NM; ++m) issue_read(m);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int m0 = (c * NM) / NC, m1 = ((c + 1) * NM) / NC;
      const int e0 = c * EPC, e1 = (c + 1) * EPC;
#pragma unroll
      for (int m = m0; m < m1; ++m) {
        if (m + RA < NM) issue_read(m + RA);
        do_mfma(m);
        // exponentials split evenly over the chunk's MFMAs
        const int ea = e0 + ((m - m0) * EPC) / (m1 - m0), eb = e0 + ((m - m0 + 1) * EPC) / (m1 - m0);
#pragma unroll
        for (int e = ea; e < eb; ++e) exp_entry(e);
      }
      if (m1 == m0) {
#pragma unroll
        for (int e = e0; e < e1; ++e) exp_entry(e);
      }
      if (c == C_K && kt + 2 < n_kt) copy_k(kt + 2);
      if (c == C_V && HAS_NEXT) copy_v(kt + 1);
    }
    if (fit_test && __any(!(ls < 65504.0f))) {
      float mxr = -INFINITY;
#pragma unroll
      for (int e = 0; e < 32; ++e) mxr = fmaxf(mxr, s_cur[e >> 4][e & 15]);
      const float m_fit = pair_max(mxr) * cs;
      const float m_new = fmaxf(m_run, m_fit);
      alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
      rescale = true;
      m_use = m_run;
      ls = 0.f;
#pragma unroll
      for (int e = 0; e < 32; ++e) exp_entry(e);
    }
    mx_next = -INFINITY;  // the row max of a tile is taken in its own step
    l_run += ls;
    if (rescale) {
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[d][r] *= alpha;
    }
    // keep the copy wait after every MFMA and read of the step
    __builtin_amdgcn_sched_barrier(0);
    wait_copies();
    if (KMASK && HAS_NEXT) kbits_cur = (uint64_t)__ballot(kbyte_next != 0);
    __syncthreads();
  };

  // ---- prologue: K(0), K(1), V(0) copied; S(0) and its row max ----
  copy_k(0);
  if (n_kt > 1) copy_k(1);
  copy_v(0);
  wait_copies();
  __syncthreads();

  f32x16 s_a[2], s_b[2];
  f16x8 pf_a[4], pf_b[4];
  float mx_a = -INFINITY, mx_b = -INFINITY;
#pragma unroll
  for (int c = 0; c < NS; ++c) {
    const int kb2 = c / KSTEPS, kk = c % KSTEPS;
    s_a[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_k(kslot(0), c), qf[kk],
                                                      kk == 0 ? f32x16{} : s_a[kb2], 0, 0, 0);
  }
#pragma unroll
  for (int e = 0; e < 32; ++e) mx_a = fmaxf(mx_a, s_a[e >> 4][e & 15]);
  __syncthreads();  // K(0) read by every wave before step 0 refills its slot

  // ---- hand-ordered steady state (head_dim 64, 4 or 8 waves, causal; dense or key-masked) ----
  // Steps [1, 1 + 2*groups) run from an asm loop (tk_attn_steps64{,_w8}.inc, made by
  // gen_attn_steps64.py) that keeps each step's 32 exponentials between its 16
  // MFMAs; every lane does the compiled step's arithmetic in the same order, so
  // the results are bit-identical.  Those steps' key tiles lie below the query
  // block (no causal mask; a key mask is applied by the _kmask loops, which
  // set invalid keys' scores to -inf) and their copies are whole tiles (K tile
  // kt+2 < S/kBN); the
  // copies use 32-bit offsets from the K and V bases (span check) and the K read
  // addresses are formed by XOR on bits 5-6 of a 256-byte-aligned row offset.
  int groups = 0;
  if constexpr (HD == 64 && (NW == 4 || NW == 8) && CAUSAL) {
    const int last = min(q0 / kBN - 1, min(n_kt, p.S / kBN) - 3);
    const int64_t span =
        ((int64_t)n_kt + 2) * max(k_tile, v_tile) * 2 + (int64_t)kBN * max(p.ks[2], p.vs[2]) * 2;
    // 32-bit unsigned offsets: only for non-negative row strides
    if (last >= 2 && p.ks[2] >= 0 && p.vs[2] >= 0 && span < (1ll << 31) && (lds_base & 255) == 0)
      groups = last / 2;
  }

  const BoolC<true> T{};
  const BoolC<false> F{};
  if (n_kt == 1) {
    step(0, s_a, s_b, pf_a, pf_b, mx_a, mx_b, F, F);
    pv_all(pf_a, vslot(0));
  } else {
    step(0, s_a, s_b, pf_a, pf_b, mx_a, mx_b, T, F);
    // Two steps per iteration with no branch between them: the loop-carried
    // accumulators then keep one register assignment.
    int kt = 1;
    if constexpr (HD == 64 && (NW == 4 || NW == 8) && CAUSAL) {
      if (groups > 0) {
        // Pinned: O^T v[64:95], Q v[96:111], the scores of tile kt v[112:143] (s_b), P of
        // tile kt-1 v[144:159] (pf_a), m_run v161, l_run v162; v160 (mx_b, no longer read
        // after the loop) holds a V read base (dense) or validity bytes (key-masked).
        static_assert(HD == 64 && kKSlots == 2 && kVSlots == 3 && TILE == 8192 && CPW * NW == 8,
                      "the generated loop's layout");
        uint32_t ko[2] = {0, 0}, vo[2] = {0, 0};  // copies per wave: 2 at 4 waves, 1 at 8
        const uint32_t kl0 = lds_base + swz_off<RB>(lane & 31, g);  // k-step kk: kl0 ^ (kk << 5)
        const uint32_t vl0 = lds_base + kKSlots * TILE + v_rd[0][0];  // V rows 8..15: +1024
        const uint32_t vl1 = lds_base + kKSlots * TILE + v_rd[0][1];
#pragma unroll
        for (int i = 0; i < CPW; ++i) {  // first copies of the loop: K(3), V(2)
          ko[i] = (uint32_t)(((int64_t)c_row[i] * p.ks[2] + k_col[i]) * 2 + 3 * k_tile * 2);
          vo[i] = (uint32_t)(((int64_t)c_row[i] * p.vs[2] + v_col[i]) * 2 + 2 * v_tile * 2);
        }
        const uint32_t ldsw = lds_base + wave * 1024;
        const uint32_t kt2 = (uint32_t)(k_tile * 2), vt2 = (uint32_t)(v_tile * 2);
        const float cs = p.scale_log2;
        uint32_t vrd = 0, vwr = 2 * TILE;  // step 1 reads V(0) from V slot 0, writes V(2) into slot 2
        uint32_t msave, cnt, flag;
#define TK_STEPS64_OUTS \
          [o0] "+{v[64:79]}"(acc_o[0]), [o1] "+{v[80:95]}"(acc_o[1]), [x0] "+{v[112:127]}"(s_b[0]), [x1] "+{v[128:143]}"(s_b[1]), \
          [w0] "+{v[144:147]}"(pf_a[0]), [w1] "+{v[148:151]}"(pf_a[1]), [w2] "+{v[152:155]}"(pf_a[2]), [w3] "+{v[156:159]}"(pf_a[3]), \
          [mxx] "+{v160}"(mx_b), [mr] "+{v161}"(m_run), [lr] "+{v162}"(l_run), [ko0] "+&v"(ko[0]), \
          [ko1] "+&v"(ko[1]), [vo0] "+&v"(vo[0]), [vo1] "+&v"(vo[1]), [vrd] "+&s"(vrd), \
          [vwr] "+&s"(vwr), [msave] "=&s"(msave), [cnt] "=&s"(cnt), [flag] "=&s"(flag)
#define TK_STEPS64_INS \
          [q0] "{v[96:99]}"(qf[0]), [q1] "{v[100:103]}"(qf[1]), [q2] "{v[104:107]}"(qf[2]), [q3] "{v[108:111]}"(qf[3]), \
          [kl0] "v"(kl0), [kl1] "v"(kl0 ^ 32u), [kl2] "v"(kl0 ^ 64u), [kl3] "v"(kl0 ^ 96u), \
          [vl0] "v"(vl0), [vl1] "v"(vl1), [kb] "s"(kb), \
          [vb] "s"(vb), [ldsw] "s"(ldsw), [kt2] "s"(kt2), [vt2] "s"(vt2), \
          [cs] "s"(cs), [groups] "s"(groups)
#define TK_STEPS64_CLOBS \
          "v163", "v164", "v165", "v166", "v167", "v168", "v169", "v170", "v171", "v172", "v173", "v174", \
          "v175", "v176", "v177", "v178", "v179", "v180", "v181", "v182", "v183", "v184", "v185", "v186", \
          "v187", "v188", "v189", "v190", "v191", "v192", "v193", "v194", "v195", "v196", "v197", "v198", \
          "v199", "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", \
          "v211", "v212", "v213", "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", \
          "v223", "v224", "v225", "v226", "v227", "v228", "v229", "vcc", "scc", "memory"
        if constexpr (KMASK) {
          // the validity byte of key 64(kt+1) + lane is read in step kt, from kt = 1
          uint32_t koff = lane + 2 * kBN;
          if constexpr (NW == 4) {
            asm volatile(
#include "tk_attn_steps64_kmask.inc"
                : TK_STEPS64_OUTS, [koff] "+&v"(koff)
                : TK_STEPS64_INS, [kvb] "s"(kvb), [kbits] "s"(kbits_cur)
                : TK_STEPS64_CLOBS, "s88", "s89", "s90", "s91", "s92", "s93", "s94", "s95");
          } else {
            asm volatile(
#include "tk_attn_steps64_w8_kmask.inc"
                : TK_STEPS64_OUTS, [koff] "+&v"(koff)
                : TK_STEPS64_INS, [kvb] "s"(kvb), [kbits] "s"(kbits_cur)
                : TK_STEPS64_CLOBS, "s88", "s89", "s90", "s91", "s92", "s93", "s94", "s95");
          }
        } else if constexpr (NW == 4) {
          asm volatile(
#include "tk_attn_steps64.inc"
              : TK_STEPS64_OUTS
              : TK_STEPS64_INS
              : TK_STEPS64_CLOBS);
        } else {
          asm volatile(
#include "tk_attn_steps64_w8.inc"
              : TK_STEPS64_OUTS
              : TK_STEPS64_INS
              : TK_STEPS64_CLOBS);
        }
#undef TK_STEPS64_OUTS
#undef TK_STEPS64_INS
#undef TK_STEPS64_CLOBS
        kt += 2 * groups;
        if constexpr (KMASK) kbits_cur = (uint64_t)__ballot(key_byte(kt) != 0);  // the loop keeps its own
      }
      // the copy addresses are rebuilt rather than kept live across the asm loop
      int ln = lane;
      asm volatile("" : "+v"(ln));
      copy_setup(ln);
    }
    for (; kt + 1 < n_kt - 1; kt += 2) {
      step(kt, s_b, s_a, pf_b, pf_a, mx_b, mx_a, T, T);
      step(kt + 1, s_a, s_b, pf_a, pf_b, mx_a, mx_b, T, T);
    }
    if (kt < n_kt - 1) step(kt, s_b, s_a, pf_b, pf_a, mx_b, mx_a, T, T);
    const int kl = n_kt - 1;
    if (kl & 1) {
      step(kl, s_b, s_a, pf_b, pf_a, mx_b, mx_a, F, T);
      pv_all(pf_b, vslot(kl % kVSlots));
    } else {
      step(kl, s_a, s_b, pf_a, pf_b, mx_a, mx_b, F, T);
      pv_all(pf_a, vslot(kl % kVSlots));
    }
  }

  // ---- normalise and store: lane holds O[row][d], d = 32*db + 8*(r/4) + 4*g + r%4 ----
  l_run = pair_sum(l_run);
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

template <int HD, int NW, bool CAUSAL, bool KMASK>
__device__ __forceinline__ void flash_vreg_body(const AttnArgs& p) {
  constexpr int BM = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int KRB = HD * 2;               // K tile row bytes
  constexpr int VRB = kBN * 2;              // V^T tile row bytes (128)
  constexpr int KSTAGE = kBN * KRB;
  constexpr int VSTAGE = HD * VRB;
  constexpr int STAGE = KSTAGE + VSTAGE;
  constexpr int K_COPIES = KSTAGE / 1024;   // 1 KB wave copies per K tile
  constexpr int K_CPW = (K_COPIES + NW - 1) / NW;
  constexpr int K_RPC = 1024 / KRB;         // K rows per copy
  constexpr int K_CPR = KRB / 16;           // 16-byte chunks per K row
  constexpr int V_BLOCKS = kBN * HD / 16;   // 4 keys x 4 dims micro-blocks
  constexpr int V_LOADS = (V_BLOCKS + NT - 1) / NT;
  constexpr int DB = (HD + 31) / 32;        // 32-row blocks of the O^T accumulator
  constexpr int KSTEPS = HD / 16;           // k16 steps of S^T = K.Q^T
  static_assert(KSTAGE % 1024 == 0, "K tile must be whole 1 KB copies");

  __shared__ __attribute__((aligned(16))) char smem[kStages * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const uint8_t* kvb = KMASK ? p.kv + b * p.kvs : nullptr;

  const int my_row = q0 + wave * 32 + (lane & 31);
  const int g = lane >> 5;
  const int wave_row_min = q0 + wave * 32;

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
  float m_run = -INFINITY;  // running max of scale*log2e*s
  float l_run = 0.f;        // lane-partial running sum (this lane's keys)

  const int kv_end = CAUSAL ? min(p.S, q0 + BM) : p.S;
  const int n_kt = (kv_end + kBN - 1) / kBN;

  // ---- K tile: direct copies; per-lane source offsets fixed, tile stride added ----
  int k_src_row[K_CPW], k_src_col[K_CPW];
#pragma unroll
  for (int i = 0; i < K_CPW; ++i) {
    const int ci = wave + i * NW;
    const int row = ci * K_RPC + lane / K_CPR;
    k_src_row[i] = row;
    k_src_col[i] = (swz_off<KRB>(row, lane % K_CPR) - row * KRB) >> 1;  // logical chunk, in halves
  }
  auto load_k = [&](int kt, int stage) {
    char* ks_ = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < K_CPW; ++i) {
      const int ci = wave + i * NW;
      if (K_COPIES % NW == 0 || ci < K_COPIES) {
        const int key = min(kt * kBN + k_src_row[i], p.S - 1);  // rows past S: finite, masked
        __builtin_amdgcn_global_load_lds(kb + (int64_t)key * p.ks[2] + k_src_col[i],
                                         (lds_void*)(ks_ + ci * 1024), 16, 0, 0);
      }
    }
  };

  // ---- V tile: 4 keys x 4 dims per thread through registers, written as V^T ----
  f16x4 rv[V_LOADS][4];
  auto load_v = [&](int kt) {
    const int k0 = kt * kBN;
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
  auto store_v = [&](int stage) {
    char* vs_ = smem + stage * STAGE + KSTAGE;
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

  // ---- S^T = K . Q^T for one tile: two 32-key blocks ----
  auto scores = [&](int stage, f32x16 (&sacc)[2]) {
    const char* ks_ = smem + stage * STAGE;
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
  };

  // ---- softmax of one tile's scores + O^T += V^T . P^T ----
  // accumulator entry r of block kb2 is key k0 + 32*kb2 + 8*(r/4) + 4*g + r%4
  // kbyte: this lane's byte of the tile's key-validity mask (key k0 + lane),
  // loaded one step ahead; the wave ballot turns it into one 64-bit word.
  auto softmax_pv = [&](int kt, int stage, f32x16 (&sacc)[2], int kbyte, bool has_next, int st_next,
                        f32x16 (&snext)[2]) {
    const int k0 = kt * kBN;
    const char* vs_ = smem + stage * STAGE + KSTAGE;
    const bool need_mask = (k0 + kBN > p.S) || (CAUSAL && k0 + kBN - 1 > wave_row_min) || KMASK;
    float mx = -INFINITY;
    if (need_mask) {
      // bit j of kbits: key k0 + 4*g + j is valid
      const uint64_t kbits = KMASK ? (uint64_t)__ballot(kbyte != 0) >> (4 * g) : 0ull;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = kb2 * 32 + 8 * (r >> 2) + (r & 3);
          const int key = k0 + j + 4 * g;
          if (key >= p.S || (CAUSAL && key > my_row) || (KMASK && ((kbits >> j) & 1) == 0))
            sacc[kb2][r] = -INFINITY;
          mx = fmaxf(mx, sacc[kb2][r]);
        }
    } else {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb2][r]);
    }
    mx = pair_max(mx);
    const float c = p.scale_log2;
    const float m_tile = mx * c;  // c > 0: max(s)*c == max(s*c)
    // Lazy rescale: the reference max m_run only moves when some row of the
    // wave has grown by more than 2^8 over it, so exponentials stay <= 256
    // (exact in fp16's range) and the O/l rescale is skipped on most tiles;
    // O and l always share one reference, so the final O/l is unchanged.
    if (__any(m_tile > m_run + 8.0f)) {
      const float m_new = fmaxf(m_run, m_tile);
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[d][r] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float ls = 0.f;
    f16x8 pf[4];
    // S^T of tile kt+1 (2 x KSTEPS MFMAs, the two key blocks alternating) in
    // the same region as this tile's 32 exponentials, K operands read RA
    // ahead; the compiler's scheduler orders the two.  (Pinning a fixed
    // MFMA/exp interleave with sched_group_barrier measured 1-3 % slower.)
    constexpr int NSM = 2 * KSTEPS;
    constexpr int RA = 3;
    const char* ks_n = smem + st_next * STAGE;
    f16x8 kfr[NSM];
    auto rd = [&](int i) {
      if (has_next)
        kfr[i] = *reinterpret_cast<const f16x8*>(ks_n + swz_off<KRB>((i & 1) * 32 + (lane & 31), 2 * (i >> 1) + g));
    };
    auto sm = [&](int i) {
      if (has_next) {
        const int kb2 = i & 1, kk = i >> 1;
        snext[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr[i], qf[kk], kk == 0 ? f32x16{} : snext[kb2], 0, 0, 0);
      }
    };
    auto ex = [&](int e) {  // entry e: block e / 16, accumulator index e % 16
      const int kb2 = e >> 4, r = e & 15;
      const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[kb2][r], c, -m_use));
      ls += pv;
      pf[kb2 * 2 + (r >> 3)][r & 7] = (f16)pv;
    };
#pragma unroll
    for (int i = 0; i < RA; ++i) rd(i);
#pragma unroll
    for (int i = 0; i < NSM; ++i) {
      if (i + RA < NSM) rd(i + RA);
      sm(i);
#pragma unroll
      for (int e = (32 * i) / NSM; e < (32 * (i + 1)) / NSM; ++e) ex(e);
    }
    l_run += ls;
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
  };

  // ---- prologue: tiles 0 and 1 resident, scores of tile 0 ----
  load_k(0, 0);
  load_v(0);
  __builtin_amdgcn_s_waitcnt(0);
  store_v(0);
  if (n_kt > 1) {
    load_k(1, 1);
    load_v(1);
    __builtin_amdgcn_s_waitcnt(0);
    store_v(1);
  }
  __syncthreads();

  f32x16 s_a[2], s_b[2];
  scores(0, s_a);

  // One step: prefetch tile kt+2, scores of kt+1 (into s_next), softmax+PV of kt.
  auto key_byte = [&](int kt) { return KMASK ? (int)kvb[min(kt * kBN + lane, p.S - 1)] : 1; };
  int kbyte_cur = key_byte(0);
  // Every step runs the softmax and P.V of its tile and the S^T of the next
  // one unconditionally (a causal tile past a wave's rows is all -inf and
  // contributes P = 0): MFMAs on conditional paths would make the register
  // allocator copy their accumulators.  HAS_NEXT is compile-time; the last
  // step is peeled.
  auto step = [&](int kt, f32x16 (&s_cur)[2], f32x16 (&s_next)[2], auto next_c) {
    constexpr bool HAS_NEXT = decltype(next_c)::value;
    const int st_cur = kt % kStages;
    const int st_nxt = (kt + 1) % kStages;
    const int st_pre = (kt + 2) % kStages;
    const bool pre = kt + 2 < n_kt;
    const int kbyte = kbyte_cur;
    if (HAS_NEXT) kbyte_cur = key_byte(kt + 1);
    if (pre) {
      load_k(kt + 2, st_pre);
      load_v(kt + 2);
    }
    softmax_pv(kt, st_cur, s_cur, kbyte, HAS_NEXT, st_nxt, s_next);
    if (pre) {
      __builtin_amdgcn_s_waitcnt(0);
      store_v(st_pre);
    }
    __syncthreads();
  };
  const BoolC<true> T{};
  const BoolC<false> F{};
  int kt = 0;
  for (; kt + 2 < n_kt; kt += 2) {
    step(kt, s_a, s_b, T);
    step(kt + 1, s_b, s_a, T);
  }
  if (kt + 1 < n_kt) {
    step(kt, s_a, s_b, T);
    step(kt + 1, s_b, s_a, F);
  } else {
    step(kt, s_a, s_b, F);
  }

  // ---- normalise and store: lane holds O[row][d], d = 32*db + 8*(r/4) + 4*g + r%4 ----
  l_run = pair_sum(l_run);
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

// ---- head_dim 128: K and V by LDS-DMA rings, P.V deferred one step ----
// Step t computes S^T(t) = K(t).Q^T, then runs the O^T MFMAs of tile t-1
// (P(t-1) from the previous step, V(t-1) by transposed LDS reads) between
// the exponentials of tile t.  No scores are computed ahead, so one score
// tile and two fp16 P tiles are live beside the 128-wide O accumulator and
// the Q fragments (about 200 registers: two waves per SIMD fit without
// spilling).  At head_dim 128 a step's P.V MFMAs (16 per wave, 512 cycles)
// cover its exponential work, so the only MFMA-idle phase of a wave is the
// row max between its S^T and P.V MFMAs, which the other wave of the SIMD
// fills.  K and V rings of three 16 KB slots: the copies of K(t+2) and
// V(t+1) are issued during step t and must land by the end of step t+1, so
// each copy has a whole step of slack beyond the step that issues it; the
// barrier at the end of a step waits only for the previous step's copies.
template <int HD, int NW, bool CAUSAL, bool KMASK>
__device__ __forceinline__ void flash_ring_body(const AttnArgs& p) {
  constexpr int BM = 32 * NW;
  constexpr int RB = HD * 2;               // K / V tile row bytes
  constexpr int CPR = RB / 16;             // 16-byte chunks per row
  constexpr int TILE = kBN * RB;           // bytes per K or V tile
  constexpr int COPIES = TILE / 1024;      // 1 KB wave copies per tile
  constexpr int CPW = COPIES / NW;         // copies per wave per tile
  constexpr int RPC = 1024 / RB;           // tile rows per copy
  constexpr int DB = HD / 32;              // 32-row blocks of the O^T accumulator
  constexpr int KSTEPS = HD / 16;          // k16 steps of S^T = K.Q^T
  constexpr int NS = 2 * KSTEPS;           // S^T MFMAs per tile
  constexpr int NP = 4 * DB;               // O^T MFMAs per tile
  constexpr int SL = 3;                    // slots per ring
  static_assert(HD % 32 == 0 && COPIES % NW == 0, "whole copies per wave");
  static_assert(32 % NP == 0 || NP % 32 == 0, "exponentials spread evenly over the P.V MFMAs");

  __shared__ __attribute__((aligned(16))) char smem[2 * SL * TILE];
  const uint32_t lds_base = (uint32_t)(size_t)(lds_char*)smem;
  auto kslot = [&](int i) { return smem + i * TILE; };
  auto vslot = [&](int i) { return smem + (SL + i) * TILE; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const uint8_t* kvb = KMASK ? p.kv + b * p.kvs : nullptr;

  const int my_row = q0 + wave * 32 + (lane & 31);
  const int g = lane >> 5;
  const int wave_row_min = q0 + wave * 32;

  f16x8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    if (my_row < p.S)
      qf[kk] = *reinterpret_cast<const f16x8*>(qb + (int64_t)my_row * p.qs[2] + kk * 16 + g * 8);
    else
      qf[kk] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  wait_copies();  // Q is in registers before any copy is issued

  f32x16 acc_o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[d][r] = 0.f;
  float m_run = -INFINITY;  // running max of scale*log2e*s
  float l_run = 0.f;        // lane-partial running sum (this lane's keys)

  const int kv_end = CAUSAL ? min(p.S, q0 + BM) : p.S;
  const int n_kt = (kv_end + kBN - 1) / kBN;

  // ---- copies (the layouts of flash_dma_body) ----
  int c_row[CPW], k_col[CPW], v_col[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int ci = wave + i * NW;
    const int row = ci * RPC + lane / CPR;
    const int phys = lane % CPR;
    c_row[i] = row;
    k_col[i] = ((swz_off<RB>(row, phys) - row * RB) >> 4) * 8;  // the XOR is an involution
    v_col[i] = (phys ^ vswz<RB>(row)) * 8;
  }
  auto copy_tile = [&](const f16* base, int64_t rs, const int (&col)[CPW], int j, uint32_t dst) {
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      // rows past S re-read row S-1 (finite; masked or multiplied by P = 0)
      const int key = min(j * kBN + c_row[i], p.S - 1);
      dma16(base + (int64_t)key * rs + col[i], dst + (wave + i * NW) * 1024);
    }
  };
  auto copy_k = [&](int j) { copy_tile(kb, p.ks[2], k_col, j, lds_base + (j % SL) * TILE); };
  auto copy_v = [&](int j) { copy_tile(vb, p.vs[2], v_col, j, lds_base + (SL + j % SL) * TILE); };

  // ---- operand reads ----
  // S^T MFMA c: key block c & 1, k-step c >> 1 (the two accumulation chains alternate)
  auto read_k = [&](const char* ks_, int c) {
    return *reinterpret_cast<const f16x8*>(ks_ + swz_off<RB>((c & 1) * 32 + (lane & 31), 2 * (c >> 1) + g));
  };
  int v_rd[2][DB];
  {
    const int tq = lane >> 4, ts = lane & 15;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const int row = 8 * r + 4 * (tq >> 1) + (ts >> 2);
        const int col = 32 * d + 16 * (tq & 1) + 4 * (ts & 3);
        v_rd[r][d] = row * RB + (((col >> 3) ^ vswz<RB>(row)) << 4) + (col & 7) * 2;
      }
  }
  auto read_v = [&](const char* vs_, int c) -> f16x8 {
    const int t = c / DB, d = c % DB;
    const lds_char* base = (const lds_char*)(vs_ + t * 16 * RB);
    const tr_f16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[0][d]));
    const tr_f16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[1][d]));
    return __builtin_shufflevector(__builtin_bit_cast(f16x4, lo), __builtin_bit_cast(f16x4, hi), 0, 1, 2, 3, 4, 5,
                                   6, 7);
  };

  auto key_byte = [&](int kt) { return KMASK ? (int)kvb[min(kt * kBN + lane, p.S - 1)] : 1; };
  uint64_t kbits_cur = KMASK ? (uint64_t)__ballot(key_byte(0) != 0) : 0ull;  // bit j: key j of the tile valid
  const auto ones = __builtin_bit_cast(hf16x2, 0x3c003c00u);
  constexpr int RA = 3;  // operand reads run this many MFMAs ahead of their use

  // One step: S^T(kt); row max; P.V of tile kt-1 interleaved with the
  // exponentials of tile kt; copies of K(kt+2) and V(kt+1).  Accumulator
  // entry r of block kb2 is key k0 + 32*kb2 + 8*(r/4) + 4*g + r%4.
  auto step = [&](int kt, f16x8 (&p_cur)[4], const f16x8 (&p_prev)[4], auto prev_c) {
    constexpr bool HAS_PREV = decltype(prev_c)::value;
    const int k0 = kt * kBN;
    const bool cp_k = kt + 2 < n_kt, cp_v = kt + 1 < n_kt;
    // the next tile's key-validity byte: loaded here, turned into bits after
    // the step's copy wait (its use would otherwise wait for the copies)
    int kbyte_next = 1;
    if (KMASK && cp_v) kbyte_next = key_byte(kt + 1);

    // ---- S^T(kt) = K(kt) . Q^T; the step's copies go out behind the first MFMAs ----
    const char* ks_ = kslot(kt % SL);
    f32x16 s[2];
    f16x8 kfr[NS];
#pragma unroll
    for (int c = 0; c < RA; ++c) kfr[c] = read_k(ks_, c);
#pragma unroll
    for (int c = 0; c < NS; ++c) {
      if (c + RA < NS) kfr[c + RA] = read_k(ks_, c + RA);
      const int kb2 = c & 1, kk = c >> 1;
      s[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr[c], qf[kk], kk == 0 ? f32x16{} : s[kb2], 0, 0, 0);
      if (c == NS / 4 && cp_k) copy_k(kt + 2);
      if (c == NS / 2 && cp_v) copy_v(kt + 1);
    }

    // ---- mask and row max ----
    float mx = -INFINITY;
    const bool need_mask = (k0 + kBN > p.S) || (CAUSAL && k0 + kBN - 1 > wave_row_min) || KMASK;
    if (need_mask) {
      // bit j of kbits: key k0 + 4*g + j is valid
      const uint64_t kbits = kbits_cur >> (4 * g);
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = kb2 * 32 + 8 * (r >> 2) + (r & 3);
          const int key = k0 + j + 4 * g;
          if (key >= p.S || (CAUSAL && key > my_row) || (KMASK && ((kbits >> j) & 1) == 0))
            s[kb2][r] = -INFINITY;
          mx = fmaxf(mx, s[kb2][r]);
        }
    } else {
#pragma unroll
      for (int e = 0; e < 32; ++e) mx = fmaxf(mx, s[e >> 4][e & 15]);
    }
    mx = pair_max(mx);
    const float cs = p.scale_log2;
    const float m_tile = mx * cs;  // cs > 0: max(s)*cs == max(s*cs)
    // Lazy rescale (as flash_dma_body): the reference max moves only when a
    // row of the wave has grown by more than 2^8 over it.  O is rescaled
    // after the deferred P.V MFMAs have added tile kt-1 at the old reference.
    const bool rescale = __any(m_tile > m_run + 8.0f);
    float alpha = 1.0f;
    if (rescale) {
      const float m_new = fmaxf(m_run, m_tile);
      alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;

    // ---- P.V(kt-1) MFMAs interleaved with the exponentials of tile kt ----
    const char* vs_p = vslot((kt + SL - 1) % SL);
    f16x8 vfr[NP];
    if (HAS_PREV) {
#pragma unroll
      for (int c = 0; c < RA; ++c) vfr[c] = read_v(vs_p, c);
    }
    float ls = 0.f;
    auto exp_pair = [&](int e) {  // entries e, e+1 (e even)
      const f16x2 hp = {(f16)__builtin_amdgcn_exp2f(fmaf(s[e >> 4][e & 15], cs, -m_use)),
                        (f16)__builtin_amdgcn_exp2f(fmaf(s[(e + 1) >> 4][(e + 1) & 15], cs, -m_use))};
      p_cur[e >> 3][e & 7] = hp[0];
      p_cur[e >> 3][(e & 7) + 1] = hp[1];
      ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(hf16x2, hp), ones, ls, false);
    };
    constexpr int EPM = 32 / NP;  // exponentials per P.V MFMA
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      if (HAS_PREV) {
        if (c + RA < NP) vfr[c + RA] = read_v(vs_p, c + RA);
        acc_o[c % DB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vfr[c], p_prev[c / DB], acc_o[c % DB], 0, 0, 0);
      }
#pragma unroll
      for (int e = c * EPM; e < (c + 1) * EPM; e += 2) exp_pair(e);
    }
    l_run += ls;
    if (rescale) {
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[d][r] *= alpha;
    }
    // ---- K(kt+1) and V(kt) (issued last step) land; this step's copies may stay in flight ----
    __builtin_amdgcn_sched_barrier(0);
    if (cp_k) wait_vmcnt<2 * CPW>();
    else if (cp_v) wait_vmcnt<CPW>();
    else wait_vmcnt<0>();
    if (KMASK && cp_v) kbits_cur = (uint64_t)__ballot(kbyte_next != 0);
    lds_barrier();
  };

  // ---- prologue: K(0), K(1), V(0) resident ----
  copy_k(0);
  if (n_kt > 1) copy_k(1);
  copy_v(0);
  wait_vmcnt<0>();
  lds_barrier();

  const BoolC<true> T{};
  const BoolC<false> F{};
  f16x8 pf_a[4], pf_b[4];
  step(0, pf_a, pf_b, F);
  int kt = 1;
  // two steps per iteration: the P buffers swap roles without register copies
  for (; kt + 1 < n_kt; kt += 2) {
    step(kt, pf_b, pf_a, T);
    step(kt + 1, pf_a, pf_b, T);
  }
  // ---- O^T += V^T . P^T of the last tile ----
  auto pv_last = [&](const f16x8(&pl)[4]) {
    const char* vs_l = vslot((n_kt - 1) % SL);
#pragma unroll
    for (int c = 0; c < NP; ++c)
      acc_o[c % DB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_v(vs_l, c), pl[c / DB], acc_o[c % DB], 0, 0, 0);
  };
  if (kt < n_kt) {
    step(kt, pf_b, pf_a, T);
    pv_last(pf_b);
  } else {
    pv_last(pf_a);
  }

  // ---- normalise and store: lane holds O[row][d], d = 32*db + 8*(r/4) + 4*g + r%4 ----
  l_run = pair_sum(l_run);
  const float inv = 1.0f / l_run;
  if (my_row < p.S) {
    f16* ob = p.o + b * p.os[0] + h * p.os[1] + (int64_t)my_row * p.os[2];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int dd = d * 32 + 8 * q + 4 * g;
        f16x4 t = {(f16)(acc_o[d][4 * q] * inv), (f16)(acc_o[d][4 * q + 1] * inv),
                   (f16)(acc_o[d][4 * q + 2] * inv), (f16)(acc_o[d][4 * q + 3] * inv)};
        *reinterpret_cast<f16x4*>(ob + dd) = t;
      }
  }
}

// ---- head_dim 128, two wave groups half a step apart ----
// The two waves sharing a SIMD (w and w + NW/2) run the same work, and with
// both in the same phase the older one wins every MFMA slot: it finishes its
// step first and idles at the barrier while the younger one runs alone
// (s_memtime per wave at the C4 shape: the older waves waited ~1450 cycles
// per ~4300-cycle step at the barrier, the younger ~180).  Here the two
// groups order a step's work differently: between two barriers the older
// group does S^T(e), max(e), P.V(e-1) with exp(e); the younger P.V(e-1),
// S^T(e), max(e), exp(e).  The younger group's exponentials then run while
// the older group issues its P.V MFMAs, and its MFMA bursts fall where the
// older group computes its row max.
// Lifetimes: K(e) and V(e-1) are read by both groups in epoch e; copies of
// K(e+2) and V(e+1) go out at the start of epoch e and are waited for at
// the end of epoch e+1 (three-slot K ring, four-slot V ring).
// O rescales: O takes the factor of max(e) right after the P.V MFMAs that
// add tile e-1, the last tile scored at the old reference.
template <int HD, int NW, bool CAUSAL, bool KMASK>
__device__ __forceinline__ void flash_pair_body(const AttnArgs& p) {
  constexpr int BM = 32 * NW;
  constexpr int RB = HD * 2;               // K / V tile row bytes
  constexpr int CPR = RB / 16;             // 16-byte chunks per row
  constexpr int TILE = kBN * RB;           // bytes per K or V tile
  constexpr int COPIES = TILE / 1024;      // 1 KB wave copies per tile
  constexpr int CPW = COPIES / NW;         // copies per wave per tile
  constexpr int RPC = 1024 / RB;           // tile rows per copy
  constexpr int DB = HD / 32;              // 32-row blocks of the O^T accumulator
  constexpr int KSTEPS = HD / 16;          // k16 steps of S^T = K.Q^T
  constexpr int NS = 2 * KSTEPS;           // S^T MFMAs per tile
  constexpr int NP = 4 * DB;               // O^T MFMAs per tile
  constexpr int KSL = 3, VSL = 4;          // ring slots
  static_assert(HD % 32 == 0 && COPIES % NW == 0 && NW % 2 == 0, "whole copies per wave, two groups");

  __shared__ __attribute__((aligned(16))) char smem[(KSL + VSL) * TILE];
  const uint32_t lds_base = (uint32_t)(size_t)(lds_char*)smem;
  auto kslot = [&](int i) { return smem + i * TILE; };
  auto vslot = [&](int i) { return smem + (KSL + i) * TILE; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int BH = p.B * p.H;
  const int n_qt = (p.S + BM - 1) / BM;
  const int id = blockIdx.x;
  const int qt = CAUSAL ? (n_qt - 1 - id / BH) : id / BH;
  const int bh = id % BH;
  const int b = bh / p.H, h = bh % p.H;
  const int q0 = qt * BM;

  const f16* qb = p.q + b * p.qs[0] + h * p.qs[1];
  const f16* kb = p.k + b * p.ks[0] + h * p.ks[1];
  const f16* vb = p.v + b * p.vs[0] + h * p.vs[1];
  const uint8_t* kvb = KMASK ? p.kv + b * p.kvs : nullptr;

  const int my_row = q0 + wave * 32 + (lane & 31);
  const int g = lane >> 5;
  const int wave_row_min = q0 + wave * 32;

  f16x8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    if (my_row < p.S)
      qf[kk] = *reinterpret_cast<const f16x8*>(qb + (int64_t)my_row * p.qs[2] + kk * 16 + g * 8);
    else
      qf[kk] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  wait_copies();  // Q is in registers before any copy is issued

  f32x16 acc_o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[d][r] = 0.f;
  float m_run = -INFINITY;  // running max of scale*log2e*s
  float l_run = 0.f;        // lane-partial running sum (this lane's keys)

  const int kv_end = CAUSAL ? min(p.S, q0 + BM) : p.S;
  const int n_kt = (kv_end + kBN - 1) / kBN;

  // ---- copies (the layouts of flash_dma_body) ----
  int c_row[CPW];
  const f16* k_src[CPW];
  const f16* v_src[CPW];
  int k_col[CPW], v_col[CPW];
  auto copy_setup = [&](int ln) {
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int ci = wave + i * NW;
      const int row = ci * RPC + ln / CPR;
      const int phys = ln % CPR;
      c_row[i] = row;
      k_col[i] = ((swz_off<RB>(row, phys) - row * RB) >> 4) * 8;  // the XOR is an involution
      v_col[i] = (phys ^ vswz<RB>(row)) * 8;
      k_src[i] = kb + (int64_t)row * p.ks[2] + k_col[i];
      v_src[i] = vb + (int64_t)row * p.vs[2] + v_col[i];
    }
  };
  copy_setup(lane);
  const int64_t k_tile = (int64_t)kBN * p.ks[2], v_tile = (int64_t)kBN * p.vs[2];
  auto copy_tile = [&](const f16* const (&src)[CPW], const f16* base, int64_t rs, int64_t tstride,
                       const int (&col)[CPW], int j, uint32_t dst) {
    if ((j + 1) * kBN <= p.S) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) dma16(src[i] + j * tstride, dst + (wave + i * NW) * 1024);
    } else {  // rows past S re-read row S-1 (finite; masked or multiplied by P = 0)
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int key = min(j * kBN + c_row[i], p.S - 1);
        dma16(base + (int64_t)key * rs + col[i], dst + (wave + i * NW) * 1024);
      }
    }
  };
  // Past the last tile the copies repeat it (same bytes into its own slot, or
  // a free one), so every epoch issues the same number and the waits stay exact.
  auto copies = [&](int e) {
    const int jk = min(e + 2, n_kt - 1), jv = min(e + 1, n_kt - 1);
    copy_tile(k_src, kb, p.ks[2], k_tile, k_col, jk, lds_base + (jk % KSL) * TILE);
    copy_tile(v_src, vb, p.vs[2], v_tile, v_col, jv, lds_base + (KSL + jv % VSL) * TILE);
  };

  // ---- operand reads ----
  auto read_k = [&](const char* ks_, int c) {  // S^T MFMA c: key block c & 1, k-step c >> 1
    return *reinterpret_cast<const f16x8*>(ks_ + swz_off<RB>((c & 1) * 32 + (lane & 31), 2 * (c >> 1) + g));
  };
  int v_rd[2][DB];
  {
    const int tq = lane >> 4, ts = lane & 15;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const int row = 8 * r + 4 * (tq >> 1) + (ts >> 2);
        const int col = 32 * d + 16 * (tq & 1) + 4 * (ts & 3);
        v_rd[r][d] = row * RB + (((col >> 3) ^ vswz<RB>(row)) << 4) + (col & 7) * 2;
      }
  }
  auto read_v = [&](const char* vs_, int c) -> f16x8 {  // O^T MFMA c: P block c / DB, head-dim block c % DB
    const int t = c / DB, d = c % DB;
    const lds_char* base = (const lds_char*)(vs_ + t * 16 * RB);
    const tr_f16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[0][d]));
    const tr_f16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[1][d]));
    return __builtin_shufflevector(__builtin_bit_cast(f16x4, lo), __builtin_bit_cast(f16x4, hi), 0, 1, 2, 3, 4, 5,
                                   6, 7);
  };
  auto key_byte = [&](int kt) { return KMASK ? (int)kvb[min(kt * kBN + lane, p.S - 1)] : 1; };
  uint64_t kbits_cur = KMASK ? (uint64_t)__ballot(key_byte(0) != 0) : 0ull;  // bit j: key j of the tile valid
  const auto ones = __builtin_bit_cast(hf16x2, 0x3c003c00u);
  constexpr int RA = 3;  // operand reads run this many MFMAs ahead of their use

  // ---- phases ----
  // S^T(e) into s.  Accumulator entry r of block kb2 is key 64e + 32*kb2 + 8*(r/4) + 4*g + r%4.
  auto scores = [&](int e, f32x16 (&s)[2]) {
    const char* ks_ = kslot(e % KSL);
    f16x8 kfr[NS];
#pragma unroll
    for (int c = 0; c < RA; ++c) kfr[c] = read_k(ks_, c);
#pragma unroll
    for (int c = 0; c < NS; ++c) {
      if (c + RA < NS) kfr[c + RA] = read_k(ks_, c + RA);
      const int kb2 = c & 1, kk = c >> 1;
      s[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr[c], qf[kk], kk == 0 ? f32x16{} : s[kb2], 0, 0, 0);
    }
  };
  // Mask and row max of S(e); moves the reference (lazy rescale, as
  // flash_dma_body) and scales l.  Returns the O factor and whether to apply it.
  auto row_max = [&](int e, f32x16 (&s)[2], float& alpha) -> bool {
    const int k0 = e * kBN;
    float mx = -INFINITY;
    const bool need_mask = (k0 + kBN > p.S) || (CAUSAL && k0 + kBN - 1 > wave_row_min) || KMASK;
    if (need_mask) {
      const uint64_t kbits = kbits_cur >> (4 * g);  // bit j: key k0 + 4*g + j is valid
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = kb2 * 32 + 8 * (r >> 2) + (r & 3);
          const int key = k0 + j + 4 * g;
          if (key >= p.S || (CAUSAL && key > my_row) || (KMASK && ((kbits >> j) & 1) == 0))
            s[kb2][r] = -INFINITY;
          mx = fmaxf(mx, s[kb2][r]);
        }
    } else {
#pragma unroll
      for (int e2 = 0; e2 < 32; ++e2) mx = fmaxf(mx, s[e2 >> 4][e2 & 15]);
    }
    mx = pair_max(mx);
    const float m_tile = mx * p.scale_log2;  // scale > 0: max(s)*c == max(s*c)
    const bool rescale = __any(m_tile > m_run + 8.0f);
    alpha = 1.0f;
    if (rescale) {
      const float m_new = fmaxf(m_run, m_tile);
      alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
    }
    return rescale;
  };
  // O^T += V^T(j) . P^T(j) (pv_on) interleaved with the exponentials of s into pn.
  auto pv_exp = [&](bool pv_on, int j, const f16x8 (&pp)[4], const f32x16 (&s)[2], f16x8 (&pn)[4]) {
    const float cs = p.scale_log2;
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    const char* vs_ = vslot(((j % VSL) + VSL) % VSL);
    f16x8 vfr[NP];
    if (pv_on) {
#pragma unroll
      for (int c = 0; c < RA; ++c) vfr[c] = read_v(vs_, c);
    }
    float ls = 0.f;
    constexpr int EPM = 32 / NP;
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      if (pv_on) {
        if (c + RA < NP) vfr[c + RA] = read_v(vs_, c + RA);
        acc_o[c % DB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vfr[c], pp[c / DB], acc_o[c % DB], 0, 0, 0);
      }
#pragma unroll
      for (int e = c * EPM; e < (c + 1) * EPM; e += 2) {
        const f16x2 hp = {(f16)__builtin_amdgcn_exp2f(fmaf(s[e >> 4][e & 15], cs, -m_use)),
                          (f16)__builtin_amdgcn_exp2f(fmaf(s[(e + 1) >> 4][(e + 1) & 15], cs, -m_use))};
        pn[e >> 3][e & 7] = hp[0];
        pn[e >> 3][(e & 7) + 1] = hp[1];
        ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(hf16x2, hp), ones, ls, false);
      }
    }
    l_run += ls;
  };
  auto pv_only = [&](int j, const f16x8 (&pp)[4]) {
    const char* vs_ = vslot(j % VSL);
#pragma unroll
    for (int c = 0; c < NP; ++c)
      acc_o[c % DB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_v(vs_, c), pp[c / DB], acc_o[c % DB], 0, 0, 0);
  };
  auto scale_o = [&](float alpha) {
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[d][r] *= alpha;
  };
  // End of epoch e: this epoch's copies may stay in flight, the previous
  // epoch's have landed; the next tile's key bits; barrier.
  auto epoch_end = [&](int e, int kbyte_next) {
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<2 * CPW>();
    if (KMASK && e + 1 < n_kt) kbits_cur = (uint64_t)__ballot(kbyte_next != 0);
    lds_barrier();
  };
  auto next_key_byte = [&](int e) { return (KMASK && e + 1 < n_kt) ? key_byte(e + 1) : 1; };

  // ---- prologue: K(0), K(1), V(0) resident ----
  copy_tile(k_src, kb, p.ks[2], k_tile, k_col, 0, lds_base);
  {
    const int j1 = min(1, n_kt - 1);
    copy_tile(k_src, kb, p.ks[2], k_tile, k_col, j1, lds_base + (j1 % KSL) * TILE);
  }
  copy_tile(v_src, vb, p.vs[2], v_tile, v_col, 0, lds_base + KSL * TILE);
  wait_vmcnt<0>();
  lds_barrier();

  f32x16 s[2];
  f16x8 pf_a[4], pf_b[4];
  const bool older = wave < NW / 2;

  // ---- hand-ordered steady state (head_dim 128, 8 waves, causal; with or without key mask) ----
  // Epochs [1, 1 + 4*groups) run from one asm loop (tk_attn_epochs.inc, made by
  // gen_attn_epochs.py), in one instruction order for every wave.  Each lane does
  // the arithmetic of the compiled epoch in the same order, so O, m and l come out
  // bit-identical; what changes is the schedule (C4 shape b4 h16 s8192: 1239-1253
  // -> 1137 us in same-box A/B runs).  With a key mask the loop is
  // tk_attn_epochs_kmask.inc: each epoch also reads its tile's validity bytes,
  // sets invalid keys' scores to -inf and, like the compiled epoch, exponentiates
  // against 0 for rows with no valid key yet.  The epochs it covers need no
  // causal or length mask (every key tile lies below q0, so below every row of
  // the workgroup) and copy only
  // whole tiles (K tile e+2 <= e_lim+1 < S/kBN), so none of the compiled epoch's
  // clamps and guards apply.  The copies use 32-bit offsets from the K and V
  // bases (span check), and the read addresses are formed by XOR on bits 5-7 of
  // a 256-byte-aligned row offset.
  int groups = 0;
  if constexpr (HD == 128 && NW == 8 && CAUSAL) {
    const int e_lim = min(q0 / kBN, min(n_kt, p.S / kBN) - 2);
    const int64_t span =
        ((int64_t)n_kt + 2) * max(k_tile, v_tile) * 2 + (int64_t)kBN * max(p.ks[2], p.vs[2]) * 2;
    // 32-bit unsigned offsets: only for non-negative row strides
    if (e_lim > 1 && p.ks[2] >= 0 && p.vs[2] >= 0 && span < (1ll << 31) && (lds_base & 255) == 0)
      groups = (e_lim - 1) / 4;
  }
  // Pinned: O^T v[64:127], Q v[128:159], P region A v[160:175] (P(0) in, P(4*groups)
  // out), m_run v192, l_run v193; the loop's other registers are clobbered.
  auto run_epochs = [&]() {
    static_assert(HD == 128 && NW == 8 && KSL == 3 && VSL == 4 && TILE == 16384 && CPW == 2,
                  "the generated loop's layout");
    uint32_t vl[DB], ko[CPW], vo[CPW];
    const uint32_t kl0 = lds_base + swz_off<RB>(lane & 31, g);  // k-step kk: kl0 ^ (kk << 5)
#pragma unroll
    for (int d = 0; d < DB; ++d) vl[d] = lds_base + KSL * TILE + v_rd[0][d];  // v_rd[1][d] = +2048
#pragma unroll
    for (int i = 0; i < CPW; ++i) {  // first copies of the loop: K(3), V(2)
      ko[i] = (uint32_t)(((int64_t)c_row[i] * p.ks[2] + k_col[i]) * 2 + 3 * k_tile * 2);
      vo[i] = (uint32_t)(((int64_t)c_row[i] * p.vs[2] + v_col[i]) * 2 + 2 * v_tile * 2);
    }
    const uint32_t ldsw = lds_base + wave * 1024;
    const uint32_t kt2 = (uint32_t)(k_tile * 2), vt2 = (uint32_t)(v_tile * 2);
    const float cs = p.scale_log2;
    const uint32_t krd0 = TILE, kwr0 = 0;  // epoch 1 reads K slot 1, writes K(3) into slot 0
    uint32_t msave, cnt, krd, kwr, flag;
#define TK_EPOCH_OUTS \
      [o0] "+{v[64:79]}"(acc_o[0]), [o1] "+{v[80:95]}"(acc_o[1]), [o2] "+{v[96:111]}"(acc_o[2]), \
      [o3] "+{v[112:127]}"(acc_o[3]), [pa0] "+{v[160:163]}"(pf_a[0]), [pa1] "+{v[164:167]}"(pf_a[1]), \
      [pa2] "+{v[168:171]}"(pf_a[2]), [pa3] "+{v[172:175]}"(pf_a[3]), [mr] "+{v192}"(m_run), \
      [lr] "+{v193}"(l_run), [ko0] "+&v"(ko[0]), [ko1] "+&v"(ko[1]), [vo0] "+&v"(vo[0]), \
      [vo1] "+&v"(vo[1]), [msave] "=&s"(msave), [cnt] "=&s"(cnt), [krd] "=&s"(krd), [kwr] "=&s"(kwr), \
      [flag] "=&s"(flag)
#define TK_EPOCH_INS \
      [q0] "{v[128:131]}"(qf[0]), [q1] "{v[132:135]}"(qf[1]), [q2] "{v[136:139]}"(qf[2]), \
      [q3] "{v[140:143]}"(qf[3]), [q4] "{v[144:147]}"(qf[4]), [q5] "{v[148:151]}"(qf[5]), \
      [q6] "{v[152:155]}"(qf[6]), [q7] "{v[156:159]}"(qf[7]), [kl0] "v"(kl0), [vl0] "v"(vl[0]), \
      [vl1] "v"(vl[1]), [vl2] "v"(vl[2]), [vl3] "v"(vl[3]), [kb] "s"(kb), [vb] "s"(vb), \
      [ldsw] "s"(ldsw), [kt2] "s"(kt2), [vt2] "s"(vt2), [cs] "s"(cs), [groups] "s"(groups), \
      [krd0] "s"(krd0), [kwr0] "s"(kwr0)
#define TK_EPOCH_CLOBS \
      "v176", "v177", "v178", "v179", "v180", "v181", "v182", "v183", "v184", "v185", "v186", "v187", \
      "v188", "v189", "v190", "v191", "v194", "v195", "v196", "v197", "v198", "v199", "v200", "v201", \
      "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", "v211", "v212", "v213", \
      "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", "v223", "v224", "v225", \
      "v226", "v227", "vcc", "scc", "memory"
    if constexpr (KMASK) {
      // the validity byte of key 64e + lane is read in epoch e, from e = 1
      uint32_t koff = lane + kBN;
      asm volatile(
#include "tk_attn_epochs_kmask.inc"
          : TK_EPOCH_OUTS, [koff] "+&v"(koff)
          : TK_EPOCH_INS, [kvb] "s"(kvb)
          : TK_EPOCH_CLOBS, "s88", "s89", "s90", "s91", "s92", "s93", "s94", "s95");
    } else {
      asm volatile(
#include "tk_attn_epochs.inc"
          : TK_EPOCH_OUTS
          : TK_EPOCH_INS
          : TK_EPOCH_CLOBS);
    }
#undef TK_EPOCH_OUTS
#undef TK_EPOCH_INS
#undef TK_EPOCH_CLOBS
  };
  // After the loop (or in its place) the copy addresses are rebuilt from an
  // opaque lane id rather than kept live across it: held there they spill.
  auto after_epochs = [&]() {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    copy_setup(ln);
  };

  if (older) {
    // epoch e: copies; S(e); max(e); P.V(e-1) with exp(e); O rescale; barrier
    auto epoch = [&](int e, f16x8 (&pc)[4], const f16x8 (&pp)[4]) {
      const int kbn = next_key_byte(e);
      copies(e);
      scores(e, s);
      float alpha;
      const bool rs = row_max(e, s, alpha);
      pv_exp(e > 0, e - 1, pp, s, pc);
      if (rs) scale_o(alpha);
      epoch_end(e, kbn);
    };
    epoch(0, pf_a, pf_b);
    int e = 1;
    if (groups > 0) {
      run_epochs();
      e += 4 * groups;
      if constexpr (KMASK) kbits_cur = (uint64_t)__ballot(key_byte(e) != 0);  // the loop keeps its own
    }
    after_epochs();
    for (; e + 1 < n_kt; e += 2) {
      epoch(e, pf_b, pf_a);
      epoch(e + 1, pf_a, pf_b);
    }
    wait_vmcnt<0>();
    if (e < n_kt) {
      epoch(e, pf_b, pf_a);
      wait_vmcnt<0>();
      pv_only(n_kt - 1, pf_b);
    } else {
      pv_only(n_kt - 1, pf_a);
    }
  } else {
    // epoch e: copies; P.V(e-1); S(e); max(e); exp(e); O rescale (O holds
    // the tiles < e, added at the old reference); barrier.  P crosses the
    // barrier, the scores do not.
    auto epoch = [&](int e, f16x8 (&pc)[4], const f16x8 (&pp)[4]) {
      const int kbn = next_key_byte(e);
      copies(e);
      if (e > 0) pv_only(e - 1, pp);
      scores(e, s);
      float alpha;
      const bool rs = row_max(e, s, alpha);
      pv_exp(false, 0, pp, s, pc);
      if (rs) scale_o(alpha);
      epoch_end(e, kbn);
    };
    epoch(0, pf_a, pf_b);
    int e = 1;
    if (groups > 0) {
      run_epochs();
      e += 4 * groups;
      if constexpr (KMASK) kbits_cur = (uint64_t)__ballot(key_byte(e) != 0);  // the loop keeps its own
    }
    after_epochs();
    for (; e + 1 < n_kt; e += 2) {
      epoch(e, pf_b, pf_a);
      epoch(e + 1, pf_a, pf_b);
    }
    wait_vmcnt<0>();
    if (e < n_kt) {
      epoch(e, pf_b, pf_a);
      wait_vmcnt<0>();
      pv_only(n_kt - 1, pf_b);
    } else {
      pv_only(n_kt - 1, pf_a);
    }
  }

  // ---- normalise and store: lane holds O[row][d], d = 32*db + 8*(r/4) + 4*g + r%4 ----
  l_run = pair_sum(l_run);
  const float inv = 1.0f / l_run;
  if (my_row < p.S) {
    f16* ob = p.o + b * p.os[0] + h * p.os[1] + (int64_t)my_row * p.os[2];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int dd = d * 32 + 8 * q + 4 * g;
        f16x4 t = {(f16)(acc_o[d][4 * q] * inv), (f16)(acc_o[d][4 * q + 1] * inv),
                   (f16)(acc_o[d][4 * q + 2] * inv), (f16)(acc_o[d][4 * q + 3] * inv)};
        *reinterpret_cast<f16x4*>(ob + dd) = t;
      }
  }
}

// ---- one key tile (S <= 64, head_dim <= 64) ----
// Short sequences are latency-bound (the reference's B256 S64 config runs
// 2048 heads of one tile each): a workgroup loads Q, one K and one V tile
// and writes O once.  This body keeps only what one tile needs -- no
// next-tile scores, no deferred P, no copy ring -- so it needs about a third
// of flash_dma_body's registers and 16 KB of LDS, and all workgroups of such
// a launch are resident at once.  For one tile the DMA body's running max is
// the tile max, so the operand layouts, the exponentials, the row sums (of the
// fp32 exponentials, as the causal DMA body) and the MFMA order here are the
// same and the results are identical.
template <int HD, int NW, bool CAUSAL, bool KMASK>
__device__ __forceinline__ void flash_single_body(const AttnArgs& p) {
  constexpr int BM = 32 * NW;
  constexpr int RB = HD * 2;               // K / V tile row bytes
  constexpr int CPR = RB / 16;             // 16-byte chunks per row
  constexpr int TILE = kBN * RB;           // bytes per K or V tile
  constexpr int COPIES = TILE / 1024;      // 1 KB wave copies per tile
  constexpr int CPW = (COPIES + NW - 1) / NW;
  constexpr int RPC = 1024 / RB;           // tile rows per copy
  constexpr int KSTEPS = HD / 16;          // k16 steps of S^T = K.Q^T
  static_assert(HD <= 64 && BM >= kBN, "one key tile, every query row in the workgroup");
  static_assert(TILE % 1024 == 0, "tiles must be whole 1 KB copies");

  __shared__ __attribute__((aligned(16))) char smem[2 * TILE];
  const uint32_t lds_base = (uint32_t)(size_t)(lds_char*)smem;
  const char* ks_ = smem;
  const char* vs_ = smem + TILE;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bh = blockIdx.x;  // one workgroup per (batch, head): S <= BM
  const int b = bh / p.H, h = bh % p.H;
  const f16* qb = p.q + b * p.qs[0] + h * p.qs[1];
  const f16* kb = p.k + b * p.ks[0] + h * p.ks[1];
  const f16* vb = p.v + b * p.vs[0] + h * p.vs[1];
  const int my_row = wave * 32 + (lane & 31);
  const int g = lane >> 5;

  // K and V tiles, row-major as in flash_dma_body (K chunk-swizzled, V with
  // the transposed-read swizzle); rows past S re-read row S-1 (finite,
  // masked or multiplied by P = 0).
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int ci = wave + i * NW;
    if (COPIES % NW == 0 || ci < COPIES) {
      const int row = ci * RPC + lane / CPR;
      const int phys = lane % CPR;
      const int key = min(row, p.S - 1);
      const int kc = ((swz_off<RB>(row, phys) - row * RB) >> 4) * 8;  // the XOR is an involution
      const int vc = (phys ^ vswz<RB>(row)) * 8;
      dma16(kb + (int64_t)key * p.ks[2] + kc, lds_base + ci * 1024);
      dma16(vb + (int64_t)key * p.vs[2] + vc, lds_base + TILE + ci * 1024);
    }
  }
  // Q^T fragments (B operand): lane supplies Q[row][16*kk + 8*g .. +8].
  f16x8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    if (my_row < p.S)
      qf[kk] = *reinterpret_cast<const f16x8*>(qb + (int64_t)my_row * p.qs[2] + kk * 16 + g * 8);
    else
      qf[kk] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  // bit j: key j is valid
  const uint64_t kbits = KMASK ? (uint64_t)__ballot(p.kv[b * p.kvs + min(lane, p.S - 1)] != 0) : 0ull;
  wait_copies();
  __syncthreads();

  attend_one_tile<HD, CAUSAL, KMASK>(ks_, vs_, qf, my_row, p.S, kbits, p.scale_log2,
                                     p.o + b * p.os[0] + h * p.os[1], p.os[2]);
}

// ---- any head_dim <= 256, any element strides and alignment ----
// Head dims without a tile of their own (e.g. 8, 24, 100) and q/k/v/out views
// whose rows are not 16-byte vectors run here, on the tile of the next
// supported width HDP (the reference pads its head-dim block the same way,
// src/kernels.py:262-263).  Q, K and V are read element by element with the
// head-dim tail past hd (and keys past S) filled with zeros, so the padded
// columns add exact zeros to Q.K^T and produce zero O^T rows that are never
// stored; no padded copy of any operand is made.  Four waves of 32 query rows,
// one 64-key tile at a time through registers into the flash_dma_body LDS
// layouts (K chunk-swizzled, V for the transposed reads), exact online
// softmax (the running max moves with every tile), O stored element-wise.
// VEC (hd == HDP, 16-byte q/k/v rows, 8-byte out rows): the same loop with
// 16-byte Q/K/V loads and 8-byte O stores -- the head_dim-256 path, where
// this plain loop fits its registers (one wave per SIMD, no spill).
template <int HDP, bool CAUSAL, bool KMASK, bool VEC>
__global__ __launch_bounds__(256) void flash_generic_kernel(AttnArgs p, int hd) {
  constexpr int NW = 4, BM = 32 * NW, NT = 64 * NW;
  constexpr int RB = HDP * 2;              // K / V tile row bytes
  constexpr int CPR = RB / 16;             // 16-byte chunks per row
  constexpr int TILE = kBN * RB;
  constexpr int DB = (HDP + 31) / 32;
  constexpr int KSTEPS = HDP / 16;
  constexpr int NP = 4 * DB;
  constexpr int LOADS = (kBN * CPR + NT - 1) / NT;  // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) char smem[2 * TILE];
  char* ks_ = smem;
  char* vs_ = smem + TILE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int BH = p.B * p.H;
  const int n_qt = (p.S + BM - 1) / BM;
  const int qt = CAUSAL ? (n_qt - 1 - (int)blockIdx.x / BH) : (int)blockIdx.x / BH;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  const int q0 = qt * BM;
  const f16* qb = p.q + b * p.qs[0] + h * p.qs[1];
  const f16* kb = p.k + b * p.ks[0] + h * p.ks[1];
  const f16* vb = p.v + b * p.vs[0] + h * p.vs[1];
  const uint8_t* kvb = KMASK ? p.kv + b * p.kvs : nullptr;
  const int my_row = q0 + wave * 32 + (lane & 31);
  const int g = lane >> 5;

  f16x8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    if constexpr (VEC) {
      qf[kk] = my_row < p.S ? *reinterpret_cast<const f16x8*>(qb + (int64_t)my_row * p.qs[2] + kk * 16 + g * 8)
                            : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int col = kk * 16 + g * 8 + e;
        qf[kk][e] = (my_row < p.S && col < hd) ? qb[(int64_t)my_row * p.qs[2] + col] : (f16)0;
      }
    }
  }

  f32x16 acc_o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[d][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  int v_rd[2][DB];
  {
    const int tq = lane >> 4, ts = lane & 15;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const int row = 8 * r + 4 * (tq >> 1) + (ts >> 2);
        const int col = 32 * d + (HDP >= 32 ? 16 * (tq & 1) : 0) + 4 * (ts & 3);
        v_rd[r][d] = row * RB + (((col >> 3) ^ vswz<RB>(row)) << 4) + (col & 7) * 2;
      }
  }
  const bool d_ok = HDP % 32 == 0 || (lane & 31) < HDP;

  const int kv_end = CAUSAL ? min(p.S, q0 + BM) : p.S;
  const int n_kt = (kv_end + kBN - 1) / kBN;
  for (int kt = 0; kt < n_kt; ++kt) {
    const int k0 = kt * kBN;
    __syncthreads();  // the previous tile's operands are no longer read
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int idx = tid + i * NT;
      if (LOADS * NT == kBN * CPR || idx < kBN * CPR) {
        const int row = idx / CPR, ch = idx % CPR;
        const int key = k0 + row;
        f16x8 kv8, vv8;
        if constexpr (VEC) {
          kv8 = vv8 = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
          if (key < p.S) {
            kv8 = *reinterpret_cast<const f16x8*>(kb + (int64_t)key * p.ks[2] + ch * 8);
            vv8 = *reinterpret_cast<const f16x8*>(vb + (int64_t)key * p.vs[2] + ch * 8);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int col = ch * 8 + e;
            const bool in = key < p.S && col < hd;
            kv8[e] = in ? kb[(int64_t)key * p.ks[2] + col] : (f16)0;
            vv8[e] = in ? vb[(int64_t)key * p.vs[2] + col] : (f16)0;
          }
        }
        *reinterpret_cast<f16x8*>(ks_ + swz_off<RB>(row, ch)) = kv8;
        *reinterpret_cast<f16x8*>(vs_ + row * RB + ((ch ^ vswz<RB>(row)) << 4)) = vv8;
      }
    }
    const uint64_t kbits = KMASK ? (uint64_t)__ballot(kvb[min(k0 + lane, p.S - 1)] != 0) >> (4 * g) : 0ull;
    __syncthreads();

    f32x16 s[2];
#pragma unroll
    for (int c = 0; c < 2 * KSTEPS; ++c) {
      const int kb2 = c / KSTEPS, kk = c % KSTEPS;
      const f16x8 kf = *reinterpret_cast<const f16x8*>(ks_ + swz_off<RB>(kb2 * 32 + (lane & 31), 2 * kk + g));
      s[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[kk], kk == 0 ? f32x16{} : s[kb2], 0, 0, 0);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = kb2 * 32 + 8 * (r >> 2) + (r & 3);
        const int key = k0 + j + 4 * g;
        if (key >= p.S || (CAUSAL && key > my_row) || (KMASK && ((kbits >> j) & 1) == 0)) s[kb2][r] = -INFINITY;
        mx = fmaxf(mx, s[kb2][r]);
      }
    mx = pair_max(mx);
    const float cs = p.scale_log2;
    const float m_new = fmaxf(m_run, mx * cs);
    const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[d][r] *= alpha;
    f16x8 pf[4];
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float pv = __builtin_amdgcn_exp2f(fmaf(s[e >> 4][e & 15], cs, -m_use));
      const f16 ph = (f16)pv;
      pf[e >> 3][e & 7] = ph;
      l_run += (float)ph;
    }
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      const int t = c / DB, d = c % DB;
      const lds_char* base = (const lds_char*)(vs_ + t * 16 * RB);
      const tr_f16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[0][d]));
      const tr_f16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_f16x4*)(base + v_rd[1][d]));
      f16x8 vf = __builtin_shufflevector(__builtin_bit_cast(f16x4, lo), __builtin_bit_cast(f16x4, hi), 0, 1, 2, 3,
                                         4, 5, 6, 7);
      if (!d_ok) vf = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      acc_o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[t], acc_o[d], 0, 0, 0);
    }
  }

  const float inv = 1.0f / pair_sum(l_run);
  if (my_row < p.S) {
    f16* ob = p.o + b * p.os[0] + h * p.os[1] + (int64_t)my_row * p.os[2];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const int dd = d * 32 + 8 * (r >> 2) + 4 * g;
        if constexpr (VEC) {
          *reinterpret_cast<f16x4*>(ob + dd) = f16x4{(f16)(acc_o[d][r] * inv), (f16)(acc_o[d][r + 1] * inv),
                                                     (f16)(acc_o[d][r + 2] * inv), (f16)(acc_o[d][r + 3] * inv)};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (dd + e < hd) ob[dd + e] = (f16)(acc_o[d][r + e] * inv);
        }
      }
  }
}

template <int HDP, bool VEC = false>
int launch_generic(const AttnArgs& p, int hd, bool causal, hipStream_t st) {
  const int64_t grid = (int64_t)((p.S + 127) / 128) * p.B * p.H;
  const dim3 g((unsigned)grid), blk(256);
  const bool km = p.kv != nullptr;
  if (causal && km)
    hipLaunchKernelGGL((flash_generic_kernel<HDP, true, true, VEC>), g, blk, 0, st, p, hd);
  else if (causal)
    hipLaunchKernelGGL((flash_generic_kernel<HDP, true, false, VEC>), g, blk, 0, st, p, hd);
  else if (km)
    hipLaunchKernelGGL((flash_generic_kernel<HDP, false, true, VEC>), g, blk, 0, st, p, hd);
  else
    hipLaunchKernelGGL((flash_generic_kernel<HDP, false, false, VEC>), g, blk, 0, st, p, hd);
  return check_launch("tk_flash_attn_fwd");
}

// Four-wave workgroups at head_dim <= 64 ask for two waves per SIMD (two
// workgroups per CU): left alone the compiler spends 280-370 registers on
// them (one wave per SIMD).  With two independent workgroups per CU one
// workgroup's prologue and epilogue overlap the other's steady state, which
// is why long sequences also run 128-row (four-wave) query tiles at these
// head dims (measured against 256-row tiles, one workgroup per CU: b8 s2048
// causal 129 -> 118 us, b2 s32768 causal 5.81 -> 5.73 ms).
template <int HD, int NW, bool CAUSAL, bool KMASK>
__global__ __launch_bounds__(NW * 64, (NW <= 4 && HD <= 64) ? 2 : 1) void flash_fwd_kernel(AttnArgs p) {
  // head_dim 128: causal launches take the DMA-ring body (C4 shape b4 s8192:
  // 1263-1295 -> 1180-1199 us in alternating same-box runs); without the
  // causal diagonal the register body stays (its ring build spills ~100 B
  // there: b2 s4096 non-causal 318-340 vs 354 us).
  if constexpr (HD == 128 && CAUSAL && NW == 8) {
    flash_pair_body<HD, NW, CAUSAL, KMASK>(p);  // C4 b4 s8192: 1268-1300 -> 1225-1263 us against the ring body
  } else if constexpr (HD == 128 && CAUSAL) {
    flash_ring_body<HD, NW, CAUSAL, KMASK>(p);
  } else if constexpr (HD == 128) {
    flash_vreg_body<HD, NW, CAUSAL, KMASK>(p);
  } else {
    flash_dma_body<HD, NW, CAUSAL, KMASK>(p);
  }
}
template <int HD, int NW, bool CAUSAL, bool KMASK>
__global__ __launch_bounds__(NW * 64, 4) void flash_single_kernel(AttnArgs p) {
  flash_single_body<HD, NW, CAUSAL, KMASK>(p);
}
template <int HD>
int launch_single(const AttnArgs& p, bool causal, hipStream_t st) {
  const dim3 g((unsigned)(p.B * p.H)), blk(2 * 64);
  const bool km = p.kv != nullptr;
  if (causal && km)
    hipLaunchKernelGGL((flash_single_kernel<HD, 2, true, true>), g, blk, 0, st, p);
  else if (causal)
    hipLaunchKernelGGL((flash_single_kernel<HD, 2, true, false>), g, blk, 0, st, p);
  else if (km)
    hipLaunchKernelGGL((flash_single_kernel<HD, 2, false, true>), g, blk, 0, st, p);
  else
    hipLaunchKernelGGL((flash_single_kernel<HD, 2, false, false>), g, blk, 0, st, p);
  return check_launch("tk_flash_attn_fwd");
}

template <int HD, int NW>
int launch_flash(const AttnArgs& p, bool causal, hipStream_t st) {
  constexpr int BM = 32 * NW;
  const int64_t n_qt = (p.S + BM - 1) / BM;
  const int64_t grid = n_qt * p.B * p.H;
  const dim3 g((unsigned)grid), blk(NW * 64);
  const bool km = p.kv != nullptr;
  if (causal && km)
    hipLaunchKernelGGL((flash_fwd_kernel<HD, NW, true, true>), g, blk, 0, st, p);
  else if (causal)
    hipLaunchKernelGGL((flash_fwd_kernel<HD, NW, true, false>), g, blk, 0, st, p);
  else if (km)
    hipLaunchKernelGGL((flash_fwd_kernel<HD, NW, false, true>), g, blk, 0, st, p);
  else
    hipLaunchKernelGGL((flash_fwd_kernel<HD, NW, false, false>), g, blk, 0, st, p);
  return check_launch("tk_flash_attn_fwd");
}

// Query rows per workgroup: at head_dim 128, 256 (8 waves sharing each K/V
// tile, one workgroup per CU) for long sequences; at head_dim <= 64, 128
// (4 waves, two workgroups per CU) up to kLongS keys and 256 beyond -- every
// query tile streams its key prefix, so halving the tile doubles that
// traffic, and past ~32k keys the kernel becomes bound by it (b32 s100000:
// 128-row tiles 16 % slower; b2 s32768: 1 % faster); fewer rows when S is
// short so no wave idles on padding rows; one key tile (S <= 64) at
// head_dim <= 64 takes flash_single_body.
constexpr int kLongS = 32768;
template <int HD>
int dispatch_flash(const AttnArgs& p, bool causal, hipStream_t st) {
  if (p.S > 128) {
    if (HD <= 64 && p.S <= kLongS) return launch_flash<HD, 4>(p, causal, st);
    return launch_flash<HD, 8>(p, causal, st);
  }
  if (p.S > 64) return launch_flash<HD, 4>(p, causal, st);
  if constexpr (HD <= 64) return launch_single<HD>(p, causal, st);
  else return launch_flash<HD, 2>(p, causal, st);
}

}  // namespace
}  // namespace tk

using namespace tk;

// The reference's rule (src/kernels.py:96-103): the head-dim block, the next
// power of two >= max(head_dim, 16), must be at most 256.
extern "C" int tk_attention_supported(int64_t head_dim) { return head_dim <= 256; }

namespace {
// Head dims with a tile of their own, whose views take the vector paths.
bool native_head_dim(int64_t hd) { return hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256; }
int64_t head_dim_block(int64_t hd) {
  int64_t b = 16;
  while (b < hd) b *= 2;
  return b;
}
}  // namespace

extern "C" int tk_flash_attn_fwd(const tk_half* q, const tk_half* k, const tk_half* v, tk_half* out,
                                 int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, const int64_t* o_strides, float scale,
                                 int causal, const uint8_t* key_valid, int64_t key_valid_stride,
                                 void* stream) {
  TK_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && o_strides, TK_ERR_ARG,
             "tk_flash_attn_fwd: null pointer");
  TK_REQUIRE(head_dim >= 0, TK_ERR_ARG, "tk_flash_attn_fwd: head_dim=%lld < 0", (long long)head_dim);
  TK_REQUIRE(tk_attention_supported(head_dim), TK_ERR_UNSUPPORTED,
             "tk_flash_attn_fwd: head_dim=%lld above 256", (long long)head_dim);
  TK_REQUIRE(batch >= 0 && heads >= 0 && seq >= 0 && batch * heads < (1ll << 31) &&
                 seq < (1ll << 30),
             TK_ERR_ARG, "tk_flash_attn_fwd: bad sizes");
  auto al = [](const void* ptr, uintptr_t a) { return ((uintptr_t)ptr % a) == 0; };
  TK_REQUIRE(al(q, 2) && al(k, 2) && al(v, 2) && al(out, 2), TK_ERR_ARG,
             "tk_flash_attn_fwd: q/k/v/out must be 2-byte aligned");
  TK_REQUIRE(key_valid == nullptr || key_valid_stride >= seq, TK_ERR_ARG,
             "tk_flash_attn_fwd: key_valid_stride=%lld < seq=%lld", (long long)key_valid_stride, (long long)seq);
  if (batch == 0 || heads == 0 || seq == 0 || head_dim == 0) return TK_OK;
  AttnArgs p{};
  p.q = reinterpret_cast<const f16*>(q);
  p.k = reinterpret_cast<const f16*>(k);
  p.v = reinterpret_cast<const f16*>(v);
  p.o = reinterpret_cast<f16*>(out);
  for (int i = 0; i < 3; ++i) {
    p.qs[i] = q_strides[i]; p.ks[i] = k_strides[i]; p.vs[i] = v_strides[i]; p.os[i] = o_strides[i];
  }
  p.kv = key_valid;
  p.kvs = key_valid_stride;
  p.B = (int)batch; p.H = (int)heads; p.S = (int)seq;
  p.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = as_stream(stream);
  const bool c = causal != 0;
  // Vector paths: q, k rows 16-byte vectors (register / LDS-DMA copies); v
  // rows 16-byte vectors where V is DMA-copied (every body but the non-causal
  // head_dim-128 one, which loads V rows 8 bytes at a time); out rows 8-byte
  // vectors.
  const bool v8 = head_dim == 128 && !c;
  bool vec = native_head_dim(head_dim) && al(q, 16) && al(k, 16) && al(v, v8 ? 8 : 16) && al(out, 8);
  for (int i = 0; i < 3; ++i)
    vec = vec && q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % (v8 ? 4 : 8) == 0 &&
          o_strides[i] % 4 == 0;
  if (vec) {
    switch (head_dim) {
      case 16: return dispatch_flash<16>(p, c, st);
      case 32: return dispatch_flash<32>(p, c, st);
      case 64: return dispatch_flash<64>(p, c, st);
      case 128: return dispatch_flash<128>(p, c, st);
      // head_dim 256: the generic kernel's plain tile loop on 16-byte rows
      // (appendix case 8, b64 s128: 41 -> 29 us against a DMA-ring body
      // that spilled 0.5-2.6 KB per lane at this width)
      default: return launch_generic<256, true>(p, 256, c, st);
    }
  }
  const int hd = (int)head_dim;
  switch (head_dim_block(head_dim)) {
    case 16: return launch_generic<16>(p, hd, c, st);
    case 32: return launch_generic<32>(p, hd, c, st);
    case 64: return launch_generic<64>(p, hd, c, st);
    case 128: return launch_generic<128>(p, hd, c, st);
    default: return launch_generic<256>(p, hd, c, st);
  }
}
