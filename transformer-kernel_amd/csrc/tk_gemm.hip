// fp16 x fp16 -> fp32 MFMA GEMMs with fused epilogues, for gfx950.
//
//   C[m, n] = epi( sum_k A[m, k] * W[n, k] + bias[n] )
//
// A is the activation [M, K] and W the nn.Linear weight [N, K]; both are
// K-contiguous, which is exactly the operand layout v_mfma_f32_32x32x16_f16
// wants (each lane feeds 8 consecutive k of one row).  The kernel computes
// the transposed product C^T = W . A^T on the matrix cores so that every lane
// ends up holding 4 consecutive n of one output row m: bias, GELU, residual
// and LayerNorm epilogues then work on 16-byte (fp32) / 8-byte (fp16)
// vectors along the row.
//
// Block tile BM x BN (256x256 with 8 waves, 128x128 with 4, 64x64 with 1),
// K-step BK with STAGES LDS buffers.  When K is a multiple of BK the K-tiles
// are copied global -> LDS with global_load_lds_dwordx4 (no register
// staging), STAGES-1 tiles in flight, one vmcnt wait + barrier per K-step;
// otherwise a register-staged path with zero fill handles the K tail.  LDS
// rows are XOR-swizzled per 256-byte bank line, so the fragment reads and
// the copies are bank-conflict free on gfx950's 64-bank LDS.  Block ids are
// remapped so that the tiles of one XCD (workgroups are dealt round-robin
// over the 8 XCDs) form a compact group of output tiles sharing A rows and
// W rows in that XCD's L2.  Whole 256x256 tiles (M, N multiples of 256, K of
// 128) run the ping-pong K loop instead (Mainloop::run_pingpong): the two
// waves of each SIMD alternate between a phase of LDS reads and copies and a
// phase of MFMAs only, so one of them always feeds the matrix core.
#include "tk_attn_tile.hpp"

namespace tk {
namespace {


typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) const f16x8 lds_f16x8;

struct GemmArgs {
  const f16* a;
  const f16* w;
  const float* bias;
  const float* resid;
  void* c;
  const float* ln_w;
  const float* ln_b;
  float* sum_out;
  const uint8_t* row_valid;  // nullable: padded rows (tk_row_mode)
  int row_mode;
  int64_t lda, ldw, ldr, ldc;
  int M, N, K;
  float eps;
  bool vec;     // output rows admit 4-wide vector stores
  bool bias16;  // bias is 16-byte aligned
  bool kvec;    // K, lda, ldw multiples of 8 and A, W 16-byte aligned: 16-byte operand loads
  int64_t w_gstride;  // grouped W rows (Mainloop WG > 0): group stride in rows
};

// LDS tile layout: rows of BK halves (BK = 64: 128 bytes = eight 16-byte
// chunks; BK = 32: 64 bytes = four chunks).  The gfx950 LDS serves a
// 16-byte-per-lane access for 16 lanes per cycle from 64 4-byte banks (one
// 256-byte line = 2 or 4 tile rows).  The chunk index is XOR-ed with the
// row's line number (mod chunks per row), so 16 consecutive rows read at one
// logical chunk (a fragment load) and the row-wise copies both touch 16
// distinct 16-byte bank groups.
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  if constexpr (BK == 64) return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3);
  else return row * 32 + ((chunk ^ ((row >> 2) & 3)) << 3);
}

// Maps the hardware block id to an output tile (tm, tn).  Consecutive
// hardware ids go to different XCDs; the remap gives each XCD a contiguous
// run of logical ids, and logical ids walk GROUP_M tile-rows at a time.
__device__ __forceinline__ void tile_of_block(int id, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int kXcd = 8, kGroupM = 8;
  const int nb = tiles_m * tiles_n;
  const int full = nb - nb % kXcd;
  if (id < full) id = (id % kXcd) * (full / kXcd) + id / kXcd;
  const int per_group = kGroupM * tiles_n;
  const int first_m = (id / per_group) * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = id % per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// threadIdx.x through an empty asm: in the persistent kernel's tile loop the
// per-lane addresses derived from it are then formed per tile instead of
// being hoisted out of the loop and kept live across it (they spilled).
__device__ __forceinline__ int laundered_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// s_waitcnt lgkmcnt(0): every LDS read of this wave has returned.
__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

// Raw buffer resource for buffer_load ... lds: base address, no stride, no
// range limit (the callers copy whole tiles only), gfx9 data format word.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 raw_buffer_rsrc(const void* base) {
  const uint64_t b = (uint64_t)base;
  return i32x4{(int32_t)__builtin_amdgcn_readfirstlane((uint32_t)b),
               (int32_t)(__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu), -1, 0x00020000};
}

// One wave's 1 KB global -> LDS copy (buffer_load_dwordx4 ... lds: lane l's
// 16 bytes from rsrc + soff + voff land at lds_addr + 16 l).  Issued as inline
// assembly, as dma16, so the compiler's wait insertion does not put a vmcnt
// wait in front of later LDS reads; M0 is saved and restored.
__device__ __forceinline__ void dma16_buf(i32x4 rsrc, uint32_t soff, uint32_t voff, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[lds]\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[so] offen lds\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [rs] "s"(rsrc), [so] "s"(__builtin_amdgcn_readfirstlane(soff)), [vo] "v"(voff),
        [lds] "s"(__builtin_amdgcn_readfirstlane(lds_addr))
      : "memory");
}

template <int V>
struct IntC {
  static constexpr int value = V;
};

// Workgroup barrier that nothing is scheduled across (the phase boundaries of
// the ping-pong K loop).
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Main loop: accumulates the (BN x BM) transposed tile into acc.
// Wave (wm, wn) owns rows n in [wn*WN, +WN) and m in [wm*WM, +WM) of the tile.
//
// DIRECT (K % BK == 0): K-tiles are copied global -> LDS with
// global_load_lds_dwordx4, which writes a wave's 64 x 16 bytes to 1 KB of
// LDS in lane order; lane l covers tile row r0 + l / (chunks per row) and
// physical chunk l % (chunks per row), and fetches the logical chunk the
// swizzle puts there.  Rows past M / N re-read the last valid row (their
// outputs are never stored).  All STAGES buffers are filled up front; after
// K-tile t has been read into registers, a wave waits (vmcnt) only for tile
// t+1's copies, one barrier, and the freed buffer starts receiving tile
// t+STAGES.  Fragments are double-buffered in registers: the reads of k-step
// s+1 are issued between the MFMAs of k-step s, and the first reads of the
// next K-tile are issued before the MFMAs of the current tile's last k-step,
// so the matrix cores keep working across the barrier.
// Staged (K tail): 16-byte register prefetch of the next tile with zero fill
// past M, N, K, two LDS buffers.
// WG > 0 (direct path only): the tile's W rows come in groups of WG rows,
// group k starting at global row n0 + k * p.w_gstride (the q, k and v rows of
// one head in the fused QKV weight); every row must exist.
// PP (direct path, 256 x 256 tiles of 4 x 2 waves, BK 64, two stages, whole
// tiles only): the ping-pong K loop, run_pingpong below.
template <int BM, int BN, int WAVES_M, int WAVES_N, int BK, int STAGES, bool DIRECT, int WG = 0, bool PP = false>
struct Mainloop {
  static constexpr int NW = WAVES_M * WAVES_N;
  static constexpr int NT = 64 * NW;
  static constexpr bool PINGPONG = PP;
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int FM = WM / 32;
  static constexpr int FN = WN / 32;
  static constexpr int CPR = BK / 8;             // 16-byte chunks per tile row
  static constexpr int RPC = 1024 / (BK * 2);    // tile rows per 1 KB wave copy
  static constexpr int A_LOADS = BM * CPR / NT;  // staged: chunks per thread per tile
  static constexpr int W_LOADS = BN * CPR / NT;
  static constexpr int A_INSTS = BM / RPC / NW;  // direct: wave copies per tile
  static constexpr int W_INSTS = BN / RPC / NW;
  static constexpr int INSTS = A_INSTS + W_INSTS;
  static constexpr int KSTEPS = BK / 16;
  static constexpr int LDS_HALVES = STAGES * (BM + BN) * BK;
  static_assert(BK == 32 || BK == 64, "BK is 32 or 64");
  static_assert(KSTEPS % 2 == 0, "even number of k-steps per K-tile");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(DIRECT || STAGES == 2, "the staged path double-buffers");
  static_assert(WG == 0 || (DIRECT && BN % WG == 0), "grouped W rows: direct path, whole groups");
  static_assert(!DIRECT || (BM % (RPC * NW) == 0 && BN % (RPC * NW) == 0), "copies must divide waves");
  static_assert(DIRECT || ((BM * CPR) % NT == 0 && (BN * CPR) % NT == 0), "chunks must divide threads");
  static_assert((STAGES - 1) * INSTS < 64, "vmcnt range");

  __device__ static void zero(f32x16 (&acc)[FN][FM]) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }

  __device__ __forceinline__ static void run(const GemmArgs& p, int m0, int n0, f16* smem, f32x16 (&acc)[FN][FM]) {
    zero(acc);
    if constexpr (PP) run_pingpong(p, m0, n0, smem, acc);
    else if constexpr (DIRECT) run_direct(p, m0, n0, smem, acc);
    else run_staged(p, m0, n0, smem, acc);
  }

  // Ping-pong K loop.  Waves w and w + 4 share a SIMD; group 0 (waves 0-3,
  // output columns 0-127 of the tile) and group 1 (waves 4-7, columns
  // 128-255) run the same sequence one phase apart, a phase being the stretch
  // between two workgroup barriers.  In its memory phase a wave reads the 24
  // fragments of one K-tile from LDS into registers and issues its 8 copies
  // (1 KB each, 4 of A rows and 4 of W rows); in its compute phase it issues
  // that K-tile's 32 MFMAs and nothing else.  While one group computes, the
  // other loads, so each SIMD has one wave feeding its matrix core.  A copy
  // holds up its wave's issue for about 64-85 cycles (the vector-memory path
  // moves ~64 B/clk per CU), so copies interleaved with a wave's MFMAs would
  // stretch its compute phase; here they all sit in memory phases:
  //   phase 2t    group 0: reads tile t (stage t&1), copies its share of
  //                        tile t+1 into stage (t+1)&1, waits for its reads;
  //               group 1: MFMAs of tile t-1;
  //   phase 2t+1  group 0: MFMAs of tile t, then waits for its copies;
  //               group 1: reads tile t, waits for them, copies its share of
  //                        tile t+2 into stage t&1 (every read of that stage is
  //                        done: group 0's before the last barrier, its own just
  //                        now), waits until only those copies are in flight.
  // Every copy of tile t+1 has landed when phase 2t+1 ends, before group 0
  // reads it in phase 2t+2.  Tile 0 and group 1's share of tile 1 are copied
  // before the loop.  Group 1 starts with one extra barrier and skips the one
  // after its last compute phase, so both groups pass 2 * nk barriers.  Per
  // accumulator the k order is run_direct's, so the results are bit-identical
  // to it.
  // The ping-pong loop's copy addressing for output tile (m0, n0): wave w's
  // copies of a K-tile.  Copy c of a wave covers 8 rows (lane / 8 within
  // them) of A (c < 4) or W; the lane fetches the logical chunk that the LDS
  // swizzle stores at physical chunk lane % 8 of its row,
  // (lane % 8) ^ ((row >> 1) & 7), which for these rows is
  // (lane % 8) ^ (4 * (c & 1) + lane / 16).
  struct PPCopies {
    static constexpr int STAGE_BYTES = BM * BK * 2;  // one operand's K-tile: 32 KB
    uint32_t lds_a, lds_w, vo_a[2], vo_w[2], row8_a, row8_w;
    i32x4 rs_a, rs_w;
    __device__ __forceinline__ PPCopies(const GemmArgs& p, int m0, int n0, f16* smem, int lane, int wave) {
      lds_a = (uint32_t)(size_t)(lds_char*)smem + wave * A_INSTS * 1024;
      lds_w = lds_a + STAGES * STAGE_BYTES;
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const uint32_t ch = (uint32_t)((lane & 7) ^ (4 * par + (lane >> 4)));
        vo_a[par] = (uint32_t)((lane >> 3) * p.lda * 2) + (ch << 4);
        vo_w[par] = (uint32_t)((lane >> 3) * p.ldw * 2) + (ch << 4);
      }
      // buffer bases: this wave's first copy row; byte offsets per copy and K-tile
      rs_a = raw_buffer_rsrc(p.a + (int64_t)(m0 + wave * A_INSTS * 8) * p.lda);
      rs_w = raw_buffer_rsrc(p.w + (int64_t)(n0 + wave * W_INSTS * 8) * p.ldw);
      row8_a = (uint32_t)(16 * p.lda);  // 8 rows, bytes
      row8_w = (uint32_t)(16 * p.ldw);
    }
    __device__ __forceinline__ void operator()(int kt, int stage) const {
#pragma unroll
      for (int c = 0; c < A_INSTS; ++c)
        dma16_buf(rs_a, c * row8_a + kt * (BK * 2), vo_a[c & 1], lds_a + stage * STAGE_BYTES + c * 1024);
#pragma unroll
      for (int c = 0; c < W_INSTS; ++c)
        dma16_buf(rs_w, c * row8_w + kt * (BK * 2), vo_w[c & 1], lds_w + stage * STAGE_BYTES + c * 1024);
    }
  };

  // K-tile 0 of output tile (m0, n0) into stage 0, this wave's share (INSTS
  // copies): issued by the persistent kernel before the previous tile's
  // output stores, so the next run_pingpong starts with it in flight.
  __device__ __forceinline__ static void pp_prefetch(const GemmArgs& p, int m0, int n0, f16* smem) {
    const int tid = laundered_tid();
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    PPCopies(p, m0, n0, smem, lane, wave)(0, 0);
  }

  // PF >= 0: K-tile 0 was prefetched into stage 0 (pp_prefetch) when
  // `prefetched`, and exactly PF vector-memory instructions of this wave were
  // issued after it (the previous tile's stores), which may stay in flight.
  template <int PF = -1>
  __device__ __forceinline__ static void run_pingpong(const GemmArgs& p, int m0, int n0, f16* smem,
                                                      f32x16 (&acc)[FN][FM], bool prefetched = false) {
    static_assert(BM == 256 && BN == 256 && WAVES_M == 4 && WAVES_N == 2 && BK == 64 && STAGES == 2 &&
                      DIRECT && WG == 0 && A_INSTS == 4 && W_INSTS == 4,
                  "ping-pong: 256 x 256 tile, 4 x 2 waves, BK 64, two stages");
    static_assert(PF < 0 || PF + INSTS < 64, "vmcnt range");
    const int tid = PF >= 0 ? laundered_tid() : (int)threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WAVES_M;
    const int grp = wave / WAVES_M;  // = wn
    const int nk = p.K / BK;  // even and at least 2 (the dispatch checks K > 0, K % 128 == 0)
    const PPCopies copies(p, m0, n0, smem, lane, wave);
    // Fragment reads: lane byte offsets of k-step kk in the wave's first A and
    // W row block of stage 0; the swizzle term depends on the row only
    // through frow (block rows are multiples of 32), so the other blocks and
    // stage 1 are constant byte offsets, folded into the ds_read immediates.
    const int frow = lane & 31;
    const int fhalf = lane >> 5;
    uint32_t ra[KSTEPS], rw[KSTEPS];
    {
      const uint32_t lds0 = (uint32_t)(size_t)(lds_char*)smem;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        ra[kk] = lds0 + 2u * (uint32_t)swz<BK>(wm * WM + frow, 2 * kk + fhalf);
        rw[kk] = lds0 + 2u * (uint32_t)(STAGES * BM * BK + swz<BK>(grp * WN + frow, 2 * kk + fhalf));
      }
    }
    f16x8 fa[KSTEPS][FM], fw[KSTEPS][FN];
    auto reads = [&](auto stage_c) {
      constexpr int stage = decltype(stage_c)::value;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
        for (int j = 0; j < FM; ++j)
          fa[kk][j] = *reinterpret_cast<const lds_f16x8*>(ra[kk] + (uint32_t)(2 * (stage * BM * BK + j * 32 * BK)));
#pragma unroll
        for (int i = 0; i < FN; ++i)
          fw[kk][i] = *reinterpret_cast<const lds_f16x8*>(rw[kk] + (uint32_t)(2 * (stage * BN * BK + i * 32 * BK)));
      }
    };
    auto mfmas = [&]() {
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
        for (int x = 0; x < FM * FN; ++x) {
          const int i = x / FM, j = x % FM;
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[kk][i], fa[kk][j], acc[i][j], 0, 0, 0);
        }
    };
    // K-tile t in stage t & 1 (compile-time: the loop runs two K-tiles per trip)
    auto iter = [&](int t, auto stage_c) {
      constexpr int stage = decltype(stage_c)::value;
      // memory phase of tile t (group 0: phase 2t, group 1: phase 2t+1)
      reads(stage_c);
      __builtin_amdgcn_sched_barrier(0);
      if (grp == 0) {
        if (t + 1 < nk) copies(t + 1, stage ^ 1);
        wait_lgkm0();  // this K-tile's reads are done before the barrier
      } else {
        wait_lgkm0();  // every read of this stage is done: it may be refilled
        if (t + 2 < nk) {
          copies(t + 2, stage);
          wait_vmcnt<INSTS>();  // this wave's share of tile t+1 has landed
        } else {
          wait_vmcnt<0>();
        }
      }
      phase_barrier();
      // compute phase of tile t
      mfmas();
      __builtin_amdgcn_sched_barrier(0);
      if (grp == 0) wait_vmcnt<0>();  // this wave's share of tile t+1 has landed
      if (grp == 0 || t + 1 < nk) phase_barrier();
    };

    // tile 0 (every wave its share) and group 1's share of tile 1; then
    // group 1 falls one phase behind
    if constexpr (PF >= 0) {
      if (!prefetched) copies(0, 0);
      if (grp == 1) {
        copies(1, 1);
        if (prefetched) wait_vmcnt<PF + INSTS>();  // the prefetched tile 0 has landed
        else wait_vmcnt<INSTS>();
      } else {
        if (prefetched) wait_vmcnt<PF>();
        else wait_vmcnt<0>();
      }
    } else {
      copies(0, 0);
      if (grp == 1) {
        copies(1, 1);
        wait_vmcnt<INSTS>();
      } else {
        wait_vmcnt<0>();
      }
    }
    phase_barrier();
    if (grp == 1) phase_barrier();
    for (int t = 0; t < nk; t += 2) {
      iter(t, IntC<0>{});
      iter(t + 1, IntC<1>{});
    }
  }

  __device__ __forceinline__ static void run_direct(const GemmArgs& p, int m0, int n0, f16* smem, f32x16 (&acc)[FN][FM]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave % WAVES_M;
    const int wn = wave / WAVES_M;
    f16* As = smem;                      // [STAGES][BM][BK]
    f16* Ws = smem + STAGES * BM * BK;   // [STAGES][BN][BK]
    const uint32_t lds_a = (uint32_t)(size_t)(lds_char*)As;
    const uint32_t lds_w = (uint32_t)(size_t)(lds_char*)Ws;
    const int nk = p.K / BK;

    const f16* ga[A_INSTS];
    const f16* gw[W_INSTS];
#pragma unroll
    for (int i = 0; i < A_INSTS; ++i) {
      const int r = (wave * A_INSTS + i) * RPC + lane / CPR;
      const int c = swz<BK>(r, lane % CPR) - r * BK;  // physical -> logical is the same XOR
      ga[i] = p.a + (int64_t)min(m0 + r, p.M - 1) * p.lda + c;
    }
#pragma unroll
    for (int i = 0; i < W_INSTS; ++i) {
      const int r = (wave * W_INSTS + i) * RPC + lane / CPR;
      const int c = swz<BK>(r, lane % CPR) - r * BK;
      if constexpr (WG > 0)
        gw[i] = p.w + (n0 + (int64_t)(r / WG) * p.w_gstride + r % WG) * p.ldw + c;
      else
        gw[i] = p.w + (int64_t)min(n0 + r, p.N - 1) * p.ldw + c;
    }
    // Wave copy c of tile kt into `stage`: copies 0..A_INSTS-1 are A rows,
    // the rest W rows, 1 KB each.
    auto copy = [&](int kt, int stage, int c) {
      if (c < A_INSTS)
        dma16(ga[c] + kt * BK, lds_a + 2 * (stage * BM * BK + (wave * A_INSTS + c) * RPC * BK));
      else
        dma16(gw[c - A_INSTS] + kt * BK,
              lds_w + 2 * (stage * BN * BK + (wave * W_INSTS + c - A_INSTS) * RPC * BK));
    };
    const int frow = lane & 31;   // fragment row within a 32-row block
    const int fhalf = lane >> 5;  // which 8-wide k half of a 16-wide k step
    f16x8 fa[2][FM], fw[2][FN];
    // Fragment r of k-step kk: r < FM reads A block r, else W block r - FM.
    auto read1 = [&](int b, int stage, int kk, int r) {
      const int ch = 2 * kk + fhalf;
      if (r < FM)
        fa[b][r] = *reinterpret_cast<const f16x8*>(As + stage * BM * BK + swz<BK>(wm * WM + r * 32 + frow, ch));
      else
        fw[b][r - FM] =
            *reinterpret_cast<const f16x8*>(Ws + stage * BN * BK + swz<BK>(wn * WN + (r - FM) * 32 + frow, ch));
    };
    auto read = [&](int b, int stage, int kk) {
#pragma unroll
      for (int r = 0; r < FM + FN; ++r) read1(b, stage, kk, r);
    };
    auto mma1 = [&](int b, int x) {  // MFMA x of a k-step: W block x / FM, A block x % FM
      const int i = x / FM, j = x % FM;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[b][i], fa[b][j], acc[i][j], 0, 0, 0);
    };
    auto mma = [&](int b) {
#pragma unroll
      for (int x = 0; x < FM * FN; ++x) mma1(b, x);
    };
    // Scheduling hint for one k-step: one fragment read after each of the
    // first FM + FN MFMAs, then the remaining MFMAs.
    auto interleave = [&]() {
#pragma unroll
      for (int x = 0; x < FM + FN; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      }
      if constexpr (FM * FN > FM + FN) __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - FM - FN, 0);
    };

#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (s < nk) {
#pragma unroll
        for (int c = 0; c < INSTS; ++c) copy(s, s, c);
      }
    if (nk >= STAGES) wait_vmcnt<(STAGES - 1) * INSTS>();
    else wait_vmcnt<0>();
    lds_barrier();
    read(0, 0, 0);
    int cur = 0;
    auto ksteps = [&]() {  // k-steps 0 .. KSTEPS-2 of the current K-tile
#pragma unroll
      for (int kk = 0; kk < KSTEPS - 1; ++kk) {
        read((kk + 1) & 1, cur, kk + 1);
        mma(kk & 1);
        interleave();
      }
    };
    // The last K-tile is peeled off: inside the loop the fresh reads of tile
    // kt+1 and the MFMAs of tile kt's last k-step share one block, so the
    // compiler's wait before those MFMAs covers only their own (already
    // complete) fragments instead of also the fresh reads.
    for (int kt = 0; kt < nk - 1; ++kt) {
      ksteps();
      wait_lgkm0();  // this K-tile's fragments are all in registers
      if (kt + STAGES - 1 < nk) wait_vmcnt<(STAGES - 2) * INSTS>();
      else wait_vmcnt<0>();
      lds_barrier();
      if (kt + STAGES < nk) {
#pragma unroll
        for (int c = 0; c < INSTS; ++c) copy(kt + STAGES, cur, c);
      }
      cur = cur + 1 == STAGES ? 0 : cur + 1;
      read(0, cur, 0);
      mma(1);
      interleave();  // the fresh reads go out between the MFMAs, not after them
    }
    if (nk > 0) {  // K = 0: no tile, the product is 0
      ksteps();
      mma(1);
    }
  }

  __device__ __forceinline__ static void run_staged(const GemmArgs& p, int m0, int n0, f16* smem, f32x16 (&acc)[FN][FM]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % WAVES_M;
    const int wn = wave / WAVES_M;
    f16* As = smem;
    f16* Ws = smem + 2 * BM * BK;
    const int nk = (p.K + BK - 1) / BK;
    f16x8 ra[A_LOADS], rw[W_LOADS];
    auto fetch = [&](int kt) {
      const int k0 = kt * BK;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        const int idx = tid + i * NT;
        const int row = idx / CPR, ch = idx % CPR;
        const int gm = m0 + row, gk = k0 + ch * 8;
        ra[i] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (gm < p.M && gk < p.K) {
          const f16* src = p.a + (int64_t)gm * p.lda + gk;
          if (p.kvec) {
            ra[i] = *reinterpret_cast<const f16x8*>(src);
          } else {  // rows not 16-byte vectors along K: element loads, zero past K
#pragma unroll
            for (int e = 0; e < 8; ++e) ra[i][e] = gk + e < p.K ? src[e] : (f16)0;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < W_LOADS; ++i) {
        const int idx = tid + i * NT;
        const int row = idx / CPR, ch = idx % CPR;
        const int gn = n0 + row, gk = k0 + ch * 8;
        rw[i] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (gn < p.N && gk < p.K) {
          const f16* src = p.w + (int64_t)gn * p.ldw + gk;
          if (p.kvec) {
            rw[i] = *reinterpret_cast<const f16x8*>(src);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) rw[i][e] = gk + e < p.K ? src[e] : (f16)0;
          }
        }
      }
    };
    auto land = [&](int stage) {
      f16* a_s = As + stage * BM * BK;
      f16* w_s = Ws + stage * BN * BK;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        const int idx = tid + i * NT;
        *reinterpret_cast<f16x8*>(a_s + swz<BK>(idx / CPR, idx % CPR)) = ra[i];
      }
#pragma unroll
      for (int i = 0; i < W_LOADS; ++i) {
        const int idx = tid + i * NT;
        *reinterpret_cast<f16x8*>(w_s + swz<BK>(idx / CPR, idx % CPR)) = rw[i];
      }
    };
    fetch(0);
    land(0);
    __syncthreads();
    const int frow = lane & 31;
    const int fhalf = lane >> 5;
    int cur = 0;
    for (int kt = 0; kt < nk; ++kt) {
      const bool more = kt + 1 < nk;
      if (more) fetch(kt + 1);
      const f16* a_s = As + cur * BM * BK;
      const f16* w_s = Ws + cur * BN * BK;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        const int ch = 2 * kk + fhalf;
        f16x8 fa[FM], fw[FN];
#pragma unroll
        for (int j = 0; j < FM; ++j)
          fa[j] = *reinterpret_cast<const f16x8*>(a_s + swz<BK>(wm * WM + j * 32 + frow, ch));
#pragma unroll
        for (int i = 0; i < FN; ++i)
          fw[i] = *reinterpret_cast<const f16x8*>(w_s + swz<BK>(wn * WN + i * 32 + frow, ch));
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[i], fa[j], acc[i][j], 0, 0, 0);
      }
      if (more) land(cur ^ 1);
      __syncthreads();
      cur ^= 1;
    }
  }
};

// Output coordinates of accumulator element (i, j, q) for this lane:
//   m = m_wave + j*32 + (lane & 31)
//   n = n_wave + i*32 + 8*q + 4*(lane >> 5) + e,  e = 0..3  (acc index 4q+e)

// Tile configuration: block tile BM x BN, wave grid WAVES_M x WAVES_N, and
// for the direct-copy path the K step and number of LDS stages.  The staged
// (K-tail) path always runs K step 64 with two stages.
template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int BK_, int STAGES_, bool PP_ = false>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int BK = BK_, STAGES = STAGES_;
  static constexpr bool PP = PP_;
  static constexpr int NT = 64 * WAVES_M_ * WAVES_N_;
  template <bool DIRECT>
  using ML = Mainloop<BM, BN, WAVES_M, WAVES_N, DIRECT ? BK : 64, DIRECT ? STAGES : 2, DIRECT, 0, PP && DIRECT>;
};

// Byte offset of 16-byte chunk `chunk` of row `row` in a row-major LDS
// staging region with CPR chunks per row: the chunk index is XOR-ed with the
// row's position inside its 256-byte bank line group, so that 16 rows written
// at one logical chunk, and the rows read back 16 bytes per lane, each hit
// distinct banks.
template <int CPR>
__device__ __forceinline__ int epi_off(int row, int chunk) {
  int f;
  if constexpr (CPR >= 16) f = row & 15;
  else f = (row / (16 / CPR)) % CPR;
  return row * CPR * 16 + ((chunk ^ f) << 4);
}

// Residual epilogue with per-row validity (padded rows, tk_row_mode): an
// internal epilogue code, picked when row_valid is given; it runs the
// residual epilogue's passes with the per-row select.
constexpr int kEpiResidRows = 3;

// Each wave stages its WM x WN fp16 result tile (in rows of 32 x JC) in its
// own LDS region, row-major, then reads it back 16 bytes per lane along rows:
// every global store then covers whole 128-byte lines instead of 16-byte
// pieces of 32 rows.  Bias and GELU are applied in fp32 before the fp16
// rounding.  The caller has made the main-loop LDS free (every read of the
// K-tile stages complete).  WHOLE: the tile lies inside M x N, the output rows
// take 16-byte stores and a given bias 16-byte loads (no bounds tests).
template <class ML, int WAVES_M, int EPI, bool WHOLE>
__device__ __forceinline__ void store_tile_lds(const GemmArgs& p, const f32x16 (&acc)[ML::FN][ML::FM], int m0,
                                               int n0, f16* smem) {
  constexpr int WM = ML::WM, WN = ML::WN, FM = ML::FM, FN = ML::FN, NW = ML::NW;
  constexpr int ROWB = WN * 2;
  constexpr int CPR = ROWB / 16;
  constexpr int LDS_BYTES = ML::LDS_HALVES * 2;
  constexpr int JC = (NW * FM * 32 * ROWB <= LDS_BYTES) ? FM : (NW * 32 * ROWB <= LDS_BYTES ? 1 : 0);
  static_assert(JC > 0 && FM % JC == 0, "staging region does not fit");
  constexpr int EPC = 8;  // elements per chunk
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int mw = m0 + (wave % WAVES_M) * WM;
  const int nw = n0 + (wave / WAVES_M) * WN;
  char* region = reinterpret_cast<char*>(smem) + wave * (JC * 32 * ROWB);
#pragma unroll
  for (int jb = 0; jb < FM; jb += JC) {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = i * 32 + 8 * q + 4 * (lane >> 5);  // 4 consecutive n of this lane
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        const int n = nw + nl;
        if (p.bias) {
          if (WHOLE || (p.bias16 && n + 3 < p.N)) {
            const f32x4 b4 = *reinterpret_cast<const f32x4*>(p.bias + n);
            bv[0] = b4[0]; bv[1] = b4[1]; bv[2] = b4[2]; bv[3] = b4[3];
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[e] = n + e < p.N ? p.bias[n + e] : 0.f;
          }
        }
#pragma unroll
        for (int jj = 0; jj < JC; ++jj) {
          const int row = jj * 32 + (lane & 31);
          const f32x16& a = acc[i][jb + jj];
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = a[4 * q + e] + bv[e];
            if constexpr (EPI == TK_EPI_BIAS_GELU) v[e] = gelu_erf(v[e]);
          }
          *reinterpret_cast<f16x4*>(region + epi_off<CPR>(row, nl / 8) + (nl % 8) * 2) =
              f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
        }
      }
    }
    asm volatile("" ::: "memory");  // LDS accesses of one wave complete in order
    constexpr int TOT = JC * 32 * CPR;
    static_assert(TOT % 64 == 0, "whole read-back passes");
    // Partial unroll: a fully unrolled read-back makes the enclosing jb loop
    // too large to unroll, and acc[i][jb + jj] would then be indexed at run
    // time, which puts the whole accumulator in scratch memory.
#pragma unroll 4
    for (int idx0 = 0; idx0 < TOT; idx0 += 64) {
      const int idx = idx0 + lane;
      const int row = idx / CPR, ch = idx % CPR;
      const int m = mw + jb * 32 + row;
      const int n = nw + ch * EPC;
      if (WHOLE || (m < p.M && n < p.N)) {
        const f16x8 d = *reinterpret_cast<const f16x8*>(region + epi_off<CPR>(row, ch));
        f16* cr = reinterpret_cast<f16*>(p.c) + (int64_t)m * p.ldc + n;
        if (WHOLE || (p.vec && n + 7 < p.N)) {
          *reinterpret_cast<f16x8*>(cr) = d;
        } else {
          for (int e = 0; e < 8 && n + e < p.N; ++e) cr[e] = d[e];
        }
      }
    }
    asm volatile("" ::: "memory");
  }
}


// The fp16 epilogue (bias, bias + GELU) of the persistent ping-pong kernel,
// whole 256 x 256 tiles: the passes of store_tile_lds one 32-row block at a
// time (8 KB per wave) in the stage-1 half of the main-loop LDS (waves 0-3 in
// A's stage 1, 4-7 in W's), so that stage 0 can take the next tile's first
// K-tile (pp_prefetch, when has_next).  The bias vectors are loaded, and
// waited for, first: a load issued after a store or after the prefetch would
// make the compiler's wait for it also wait for those (the vector memory
// counter retires in order).  Then the prefetch, then the passes with their
// kPfStores output stores, all of which may stay in flight into the next tile.
constexpr int kPfStores = 16;
template <class ML, int WAVES_M, int EPI>
__device__ __forceinline__ void store_tile_lds_pf(const GemmArgs& p, const f32x16 (&acc)[ML::FN][ML::FM], int m0,
                                                  int n0, f16* smem, bool has_next, int next_m0, int next_n0) {
  constexpr int WM = ML::WM, WN = ML::WN, FM = ML::FM, FN = ML::FN;
  constexpr int ROWB = WN * 2;
  constexpr int CPR = ROWB / 16;
  constexpr int EPC = 8;  // elements per chunk
  constexpr int TOT = 32 * CPR;
  static_assert(ML::PINGPONG && WAVES_M == 4 && ROWB == 256 && TOT % 64 == 0, "256 x 256 ping-pong tile");
  static_assert(FM * (TOT / 64) == kPfStores, "store count after the prefetch");
  const int tid = laundered_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int mw = m0 + (wave % WAVES_M) * WM;
  const int nw = n0 + (wave / WAVES_M) * WN;
  // stage 1: A at 32 KB, W at 96 KB; 8 KB (32 rows x 256 bytes) per wave
  char* region = reinterpret_cast<char*>(smem) + (wave < 4 ? 32768 + wave * 8192 : 98304 + (wave - 4) * 8192);
  f32x4 bias[FN][4];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      bias[i][q] = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + nw + i * 32 + 8 * q + 4 * (lane >> 5))
                          : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" ::"v"(bias[i][q]));  // the loads have returned here
  if (has_next) ML::pp_prefetch(p, next_m0, next_n0, smem);
#pragma unroll
  for (int jb = 0; jb < FM; ++jb) {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = i * 32 + 8 * q + 4 * (lane >> 5);  // 4 consecutive n of this lane
        const f32x4 b4 = bias[i][q];
        const int row = lane & 31;
        const f32x16& a = acc[i][jb];
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = a[4 * q + e] + b4[e];
          if constexpr (EPI == TK_EPI_BIAS_GELU) v[e] = gelu_erf(v[e]);
        }
        *reinterpret_cast<f16x4*>(region + epi_off<CPR>(row, nl / 8) + (nl % 8) * 2) =
            f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
      }
    }
    asm volatile("" ::: "memory");  // LDS accesses of one wave complete in order
#pragma unroll
    for (int idx0 = 0; idx0 < TOT; idx0 += 64) {
      const int idx = idx0 + lane;
      const int row = idx / CPR, ch = idx % CPR;
      const int m = mw + jb * 32 + row;
      const int n = nw + ch * EPC;
      const f16x8 d = *reinterpret_cast<const f16x8*>(region + epi_off<CPR>(row, ch));
      *reinterpret_cast<f16x8*>(reinterpret_cast<f16*>(p.c) + (int64_t)m * p.ldc + n) = d;
    }
    asm volatile("" ::: "memory");
  }
}

// One pass of the fp32 residual epilogue over accumulator blocks
// [JB, JB + JC) of a wave:  C[m, n] = resid[m, n] + (acc + bias[n])  (C may
// alias resid: every element is read and written by the same lane).  The
// residual rows a lane combines (16 rows of 16 bytes per pass) are loaded
// in groups of G with one wait per group: all 16 at once, issued before the
// accumulators are staged in LDS, when the accumulator blocks still live in
// the pass leave room (at most 128 registers; 64 with padded rows, whose
// row-bit handling needs the rest), else 8 after the staging.  On the
// 256x256 tile the early group takes the kernel to 252 VGPRs at two waves
// per SIMD, without scratch.  In the row-major read-back a lane always
// lands on the same 16-byte column chunk (64 lanes cover 64 / CPR whole
// rows), so its bias is one vector.  With padded rows (ROWS: row_valid
// given) the pass's JC * 32 validity bytes are loaded once, one per lane, and
// their ballot is a wave-uniform bit mask; a lane tests its row's bit, and
// an invalid row is written as resid (TK_ROWS_KEEP_RESID) or 0.
template <class ML, int WAVES_M, int JB, int JC, bool ROWS, bool WHOLE>
__device__ __forceinline__ void resid_pass(const GemmArgs& p, const f32x16 (&acc)[ML::FN][ML::FM], int mw, int nw,
                                           char* region) {
  constexpr int FN = ML::FN;
  constexpr int CPR = ML::WN * 4 / 16;  // 16-byte chunks per staged row
  constexpr int RPI = 64 / CPR;         // staged rows per read-back step of the wave
  constexpr int NIT = JC * 32 / RPI;    // read-back steps of the pass
  constexpr bool EARLY = FN * (ML::FM - JB) * 16 <= (ROWS ? 64 : 128);
  constexpr int G = EARLY ? NIT : NIT / 2;  // rows per load group
  static_assert(64 % CPR == 0 && (JC * 32) % RPI == 0 && NIT % G == 0, "whole rows per read-back step");
  const int lane = threadIdx.x & 63;
  const int ch = lane % CPR, row0 = lane / CPR;
  const int n = nw + ch * 4;
  const bool vec = WHOLE || (p.vec && n + 3 < p.N);
  const int mb = mw + JB * 32;  // first row of the pass (wave-uniform)
  // wave-uniform base + 32-bit lane offsets (a pass spans 32 rows)
  const float* rbase = p.resid + (int64_t)mb * p.ldr + nw;
  const uint32_t ldr = (uint32_t)p.ldr;
  uint64_t rows_ok = ~0ull;  // bit r: row mb + r is valid
  const bool keep = p.row_mode == TK_ROWS_KEEP_RESID;
  static_assert(JC * 32 <= 64, "one validity bit per lane");
  if constexpr (ROWS) {
    const int m = mb + lane;
    rows_ok = __ballot(lane < JC * 32 && m < p.M && p.row_valid[m] != 0);
  }

  f32x4 r[G];
  auto fetch = [&](int g) {
#pragma unroll
    for (int it = 0; it < G; ++it) {
      const int row = (g * G + it) * RPI + row0;
      r[it] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (vec && (WHOLE || mb + row < p.M)) r[it] = *reinterpret_cast<const f32x4*>(rbase + ((uint32_t)row * ldr + ch * 4));
    }
  };
  auto combine = [&](int g, const f32x4& b) {
#pragma unroll
    for (int it = 0; it < G; ++it) {
      const int row = (g * G + it) * RPI + row0;
      const int m = mb + row;
      if (WHOLE || (m < p.M && n < p.N)) {
        const f32x4 d = *reinterpret_cast<const f32x4*>(region + epi_off<CPR>(row, ch));
        float* cr = reinterpret_cast<float*>(p.c) + (int64_t)m * p.ldc + n;
        const bool valid = !ROWS || ((rows_ok >> row) & 1ull);
        if (vec) {
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = valid ? r[it][e] + (d[e] + b[e]) : (keep ? r[it][e] : 0.f);
          *reinterpret_cast<f32x4*>(cr) = o;
        } else {
          const float* rr = p.resid + (int64_t)m * p.ldr + n;
          for (int e = 0; e < 4 && n + e < p.N; ++e)
            cr[e] = valid ? rr[e] + (d[e] + (p.bias ? p.bias[n + e] : 0.f)) : (keep ? rr[e] : 0.f);
        }
      }
    }
  };

  f32x4 b = {0.f, 0.f, 0.f, 0.f};
  if (p.bias && vec) {
    if (WHOLE || p.bias16) b = *reinterpret_cast<const f32x4*>(p.bias + n);
    else b = f32x4{p.bias[n], p.bias[n + 1], p.bias[n + 2], p.bias[n + 3]};
  }
  if constexpr (EARLY) fetch(0);
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = i * 32 + 8 * q + 4 * (lane >> 5);  // 4 consecutive n of this lane
#pragma unroll
      for (int jj = 0; jj < JC; ++jj) {
        const f32x16& a = acc[i][JB + jj];
        *reinterpret_cast<f32x4*>(region + epi_off<CPR>(jj * 32 + (lane & 31), nl / 4)) =
            f32x4{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
      }
    }
  asm volatile("" ::: "memory");  // LDS accesses of one wave complete in order
  if constexpr (!EARLY) fetch(0);
  combine(0, b);
#pragma unroll
  for (int g = 1; g < NIT / G; ++g) {
    fetch(g);
    combine(g, b);
  }
  asm volatile("" ::: "memory");
}

// fp32 residual epilogue: one resid_pass per group of JC accumulator blocks
// (two groups when the staging region holds one 32-row block per wave).  The
// caller has made the main-loop LDS free.
template <class ML, int WAVES_M, bool ROWS, bool WHOLE>
__device__ __forceinline__ void store_tile_resid(const GemmArgs& p, const f32x16 (&acc)[ML::FN][ML::FM], int m0,
                                                 int n0, f16* smem) {
  constexpr int FM = ML::FM, NW = ML::NW;
  constexpr int ROWB = ML::WN * 4;
  constexpr int LDS_BYTES = ML::LDS_HALVES * 2;
  constexpr int JC = (NW * FM * 32 * ROWB <= LDS_BYTES) ? FM : (NW * 32 * ROWB <= LDS_BYTES ? 1 : 0);
  static_assert(JC > 0 && FM % JC == 0 && FM / JC <= 2, "staging region does not fit");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int mw = m0 + (wave % WAVES_M) * ML::WM;
  const int nw = n0 + (wave / WAVES_M) * ML::WN;
  char* region = reinterpret_cast<char*>(smem) + wave * (JC * 32 * ROWB);
  resid_pass<ML, WAVES_M, 0, JC, ROWS, WHOLE>(p, acc, mw, nw, region);
  if constexpr (JC < FM) resid_pass<ML, WAVES_M, JC, JC, ROWS, WHOLE>(p, acc, mw, nw, region);
}

// The fp32 residual epilogue (dense rows) of the persistent ping-pong kernel,
// whole 256 x 256 tiles.  Four passes per wave, each over 32 rows x 64
// columns (pass k: accumulator row block k / 2, column half k % 2), staged as
// 8 KB per wave in the stage-1 half of the main-loop LDS (waves 0-3 in A's
// stage 1, 4-7 in W's), so that stage 0 can take the next tile's first
// K-tile.  Order of this wave's vector-memory instructions: bias loads
// (waited for), the prefetch (when has_next), residual rows of pass 0, then
// per pass k the residual rows of pass k + 1 before the output stores of
// pass k.  A residual wait so never covers an output store issued before
// it (the vector memory counter retires in order), the prefetch precedes
// every residual load the compiler waits for, and the last kPfStores
// instructions are the output stores of passes 2 and 3, which may stay in
// flight into the next tile.  Per element the sum is resid + (acc + bias),
// as in resid_pass, so the outputs are bit-identical to gemm_kernel's.
template <class ML, int WAVES_M>
__device__ __forceinline__ void store_tile_resid_pf(const GemmArgs& p, const f32x16 (&acc)[ML::FN][ML::FM], int m0,
                                                    int n0, f16* smem, bool has_next, int next_m0, int next_n0) {
  constexpr int FM = ML::FM, FN = ML::FN;
  constexpr int CPR = 16;          // 16-byte chunks per staged row (64 fp32)
  constexpr int RPI = 64 / CPR;    // rows per read-back step
  constexpr int NIT = 32 / RPI;    // read-back steps (residual loads) per pass
  constexpr int PASSES = FM * 2;
  static_assert(ML::PINGPONG && WAVES_M == 4 && FM == 2 && FN == 4 && ML::WN == 128, "256 x 256 ping-pong tile");
  static_assert(NIT * 2 == kPfStores, "output stores of the last two passes");
  const int tid = laundered_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int mw = m0 + (wave % WAVES_M) * ML::WM;
  const int nw = n0 + (wave / WAVES_M) * ML::WN;
  char* region = reinterpret_cast<char*>(smem) + (wave < 4 ? 32768 + wave * 8192 : 98304 + (wave - 4) * 8192);
  const int ch = lane % CPR, row0 = lane / CPR;
  f32x4 bias[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    bias[h] = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + nw + h * 64 + ch * 4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 2; ++h) asm volatile("" ::"v"(bias[h]));  // the loads have returned here
  if (has_next) ML::pp_prefetch(p, next_m0, next_n0, smem);
  const uint32_t ldr = (uint32_t)p.ldr;
  f32x4 r[2][NIT];
  auto fetch = [&](int k, f32x4 (&rk)[NIT]) {
    const float* rbase = p.resid + (int64_t)(mw + (k >> 1) * 32) * p.ldr + nw + (k & 1) * 64;
#pragma unroll
    for (int it = 0; it < NIT; ++it)
      rk[it] = *reinterpret_cast<const f32x4*>(rbase + ((uint32_t)(it * RPI + row0) * ldr + ch * 4));
  };
  auto stage = [&](int k) {
    const int jb = k >> 1, h = k & 1;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x16& a = acc[2 * h + ii][jb];
        const int chunk = ii * 8 + 2 * q + (lane >> 5);  // 4 consecutive columns of this lane
        *reinterpret_cast<f32x4*>(region + epi_off<CPR>(lane & 31, chunk)) =
            f32x4{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
      }
  };
  auto combine = [&](int k, const f32x4 (&rk)[NIT]) {
    const f32x4 b = bias[k & 1];
    float* cbase = reinterpret_cast<float*>(p.c) + (int64_t)(mw + (k >> 1) * 32) * p.ldc + nw + (k & 1) * 64;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int row = it * RPI + row0;
      const f32x4 d = *reinterpret_cast<const f32x4*>(region + epi_off<CPR>(row, ch));
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = rk[it][e] + (d[e] + b[e]);
      *reinterpret_cast<f32x4*>(cbase + (int64_t)row * p.ldc + ch * 4) = o;
    }
  };
  fetch(0, r[0]);
  stage(0);
  asm volatile("" ::: "memory");  // LDS accesses of one wave complete in order
#pragma unroll
  for (int k = 0; k < PASSES; ++k) {
    if (k + 1 < PASSES) fetch(k + 1, r[(k + 1) & 1]);
    asm volatile("" ::: "memory");  // the next pass's residual loads before this pass's stores
    combine(k, r[k & 1]);
    asm volatile("" ::: "memory");
    if (k + 1 < PASSES) stage(k + 1);
    asm volatile("" ::: "memory");
  }
}

template <class T, int EPI, bool DIRECT>
__global__ __launch_bounds__(T::NT) void gemm_kernel(GemmArgs p) {
  constexpr int BM = T::BM, BN = T::BN;
  using ML = typename T::template ML<DIRECT>;
  __shared__ __attribute__((aligned(16))) f16 smem[ML::LDS_HALVES];
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, tm, tn);
  f32x16 acc[ML::FN][ML::FM];
  ML::run(p, tm * BM, tn * BN, smem, acc);
  // The epilogues stage each wave's results in its own part of the main-loop
  // LDS.  The two-stage loop needs a barrier first (other waves may still read
  // the last K-tile); after the ping-pong loop every read of the stages has
  // completed before group 0's last barrier, so group 0 starts its epilogue
  // while group 1 issues the last K-tile's MFMAs.
  if constexpr (!ML::PINGPONG) __syncthreads();
  if constexpr (EPI == TK_EPI_BIAS_RESID || EPI == kEpiResidRows)
    store_tile_resid<ML, T::WAVES_M, EPI == kEpiResidRows, ML::PINGPONG>(p, acc, tm * BM, tn * BN, smem);
  else
    store_tile_lds<ML, T::WAVES_M, EPI, ML::PINGPONG>(p, acc, tm * BM, tn * BN, smem);
}

// Persistent ping-pong GEMM (whole 256 x 256 tiles; fp16 epilogues and the
// dense fp32 residual epilogue): block b runs tiles b, b + gridDim.x, ...
// (one XCD each, as tile_of_block expects).  Before a tile's output stores it
// copies the next tile's first K-tile into stage 0, so the next K loop
// neither waits for that copy's latency nor for the stores to drain (its
// first waits leave them in flight).  Between tiles one barrier after an
// LDS-only wait: every wave's staging reads of stage 1 are done before group
// 1 refills it; the output stores stay in flight.
template <class T, int EPI>
__global__ __launch_bounds__(T::NT) void gemm_pf_kernel(GemmArgs p) {
  constexpr int BM = T::BM, BN = T::BN;
  using ML = typename T::template ML<true>;
  static_assert(ML::PINGPONG && (EPI == TK_EPI_BIAS || EPI == TK_EPI_BIAS_GELU || EPI == TK_EPI_BIAS_RESID),
                "bias, GELU or dense residual epilogue, ping-pong loop");
  __shared__ __attribute__((aligned(16))) f16 smem[ML::LDS_HALVES];
  const int tiles_m = p.M / BM, tiles_n = p.N / BN;
  const int tiles = tiles_m * tiles_n;
  bool prefetched = false;
  for (int id = blockIdx.x; id < tiles; id += gridDim.x) {
    int tm, tn;
    tile_of_block(id, tiles_m, tiles_n, tm, tn);
    const int next = id + (int)gridDim.x;
    int ntm = 0, ntn = 0;
    if (next < tiles) tile_of_block(next, tiles_m, tiles_n, ntm, ntn);
    f32x16 acc[ML::FN][ML::FM];
    ML::zero(acc);
    ML::template run_pingpong<kPfStores>(p, tm * BM, tn * BN, smem, acc, prefetched);
    if constexpr (EPI == TK_EPI_BIAS_RESID)
      store_tile_resid_pf<ML, T::WAVES_M>(p, acc, tm * BM, tn * BN, smem, next < tiles, ntm * BM, ntn * BN);
    else
      store_tile_lds_pf<ML, T::WAVES_M, EPI>(p, acc, tm * BM, tn * BN, smem, next < tiles, ntm * BM, ntn * BN);
    wait_lgkm0();
    phase_barrier();
    prefetched = next < tiles;
  }
}

// Full-row variant: BN == N, so each block owns complete output rows and
// finishes the residual add + LayerNorm + cast before anything leaves the
// chip.  Row statistics: per-lane partial sums over its n values, the
// lane-pair exchange (lanes l and l^32 hold the two n halves of each 8-wide
// group), then across the WAVES_N waves through LDS.  Two passes (mean, then
// mean of squared deviations) on register-resident values.
template <class T, bool H_HALF, bool DIRECT>
__global__ __launch_bounds__(T::NT) void gemm_ln_kernel(GemmArgs p) {
  constexpr int BM = T::BM, WAVES_M = T::WAVES_M, WAVES_N = T::WAVES_N;
  using ML = typename T::template ML<DIRECT>;
  __shared__ __attribute__((aligned(16))) f16 smem[ML::LDS_HALVES];
  __shared__ float red[WAVES_N][BM];
  const int tiles_m = (p.M + BM - 1) / BM;
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, 1, tm, tn);
  const int m0 = tm * BM;

  f32x16 acc[ML::FN][ML::FM];
  ML::run(p, m0, 0, smem, acc);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int ml = wm * ML::WM + (lane & 31);  // tile-local row of fragment j=0
  const int n_w = wn * ML::WN + 4 * (lane >> 5);

  // s = resid + acc + bias, kept in acc.  A padded row (row_valid) takes
  // s = resid (TK_ROWS_KEEP_RESID) or s = 0.
  bool valid[ML::FM];
#pragma unroll
  for (int j = 0; j < ML::FM; ++j) {
    const int m = m0 + ml + j * 32;
    valid[j] = p.row_valid == nullptr || (m < p.M && p.row_valid[m] != 0);
  }
  const bool keep = p.row_mode == TK_ROWS_KEEP_RESID;
#pragma unroll
  for (int i = 0; i < ML::FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n_w + i * 32 + 8 * q;
      const f32x4 bv = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + n) : f32x4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < ML::FM; ++j) {
        const int m = m0 + ml + j * 32;
        f32x4 r = {0, 0, 0, 0};
        if (m < p.M) r = *reinterpret_cast<const f32x4*>(p.resid + (int64_t)m * p.ldr + n);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[i][j][4 * q + e] = valid[j] ? acc[i][j][4 * q + e] + (bv[e] + r[e]) : (keep ? r[e] : 0.f);
      }
    }

  // Row statistics, one row per (j, lane & 31).
  float mean[ML::FM], rstd[ML::FM];
#pragma unroll
  for (int j = 0; j < ML::FM; ++j) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < ML::FN; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) t += acc[i][j][r];
    t += __shfl_xor(t, 32);
    if (lane < 32) red[wn][ml + j * 32] = t;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < ML::FM; ++j) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES_N; ++w) t += red[w][ml + j * 32];
    mean[j] = t / (float)p.N;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < ML::FM; ++j) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < ML::FN; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float d = acc[i][j][r] - mean[j];
        t += d * d;
      }
    t += __shfl_xor(t, 32);
    if (lane < 32) red[wn][ml + j * 32] = t;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < ML::FM; ++j) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES_N; ++w) t += red[w][ml + j * 32];
    rstd[j] = 1.0f / sqrtf(t / (float)p.N + p.eps);
  }

#pragma unroll
  for (int i = 0; i < ML::FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n_w + i * 32 + 8 * q;
      const f32x4 gw = *reinterpret_cast<const f32x4*>(p.ln_w + n);
      const f32x4 gb = *reinterpret_cast<const f32x4*>(p.ln_b + n);
#pragma unroll
      for (int j = 0; j < ML::FM; ++j) {
        const int m = m0 + ml + j * 32;
        if (m >= p.M) continue;
        float s[4], h[4];
        const bool zero_h = !valid[j] && p.row_mode == TK_ROWS_ZERO_ALL;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[e] = acc[i][j][4 * q + e];
          h[e] = zero_h ? 0.f : (s[e] - mean[j]) * rstd[j] * gw[e] + gb[e];
        }
        if (p.sum_out)
          *reinterpret_cast<f32x4*>(p.sum_out + (int64_t)m * p.N + n) = f32x4{s[0], s[1], s[2], s[3]};
        if constexpr (H_HALF) {
          *reinterpret_cast<f16x4*>(reinterpret_cast<f16*>(p.c) + (int64_t)m * p.N + n) =
              f16x4{(f16)h[0], (f16)h[1], (f16)h[2], (f16)h[3]};
        } else {
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.c) + (int64_t)m * p.N + n) =
              f32x4{h[0], h[1], h[2], h[3]};
        }
      }
    }
}

template <class T, int EPI>
int launch_gemm(const GemmArgs& p, hipStream_t st) {
  const int64_t tiles = (int64_t)((p.M + T::BM - 1) / T::BM) * ((p.N + T::BN - 1) / T::BN);
  // The direct global->LDS copy needs whole K tiles of 16-byte row chunks.
  if (p.K % T::BK == 0 && p.kvec) {
    hipLaunchKernelGGL((gemm_kernel<T, EPI, true>), dim3((unsigned)tiles), dim3(T::NT), 0, st, p);
  } else {
    hipLaunchKernelGGL((gemm_kernel<T, EPI, false>), dim3((unsigned)tiles), dim3(T::NT), 0, st, p);
  }
  return check_launch("tk_gemm");
}

using TileBig = Tile<256, 256, 4, 2, 64, 2>;   // 8 waves of 64 x 128
using TileBigPP = Tile<256, 256, 4, 2, 64, 2, true>;  // the same, ping-pong K loop (whole tiles)
using TileMid = Tile<128, 128, 2, 2, 64, 2>;   // 4 waves of 64 x 64, 2 blocks per CU
using TileSmall = Tile<64, 64, 1, 1, 64, 2>;   // 1 wave

#ifndef TK_GEMM_PF
#define TK_GEMM_PF 1
#endif
constexpr bool kGemmPf = TK_GEMM_PF;
constexpr int kPfGrid = 256;  // one persistent workgroup per CU

template <int EPI>
int gemm_dispatch(const GemmArgs& p, hipStream_t st) {
  const int64_t t256 = (int64_t)((p.M + 255) / 256) * ((p.N + 255) / 256);
  const int64_t t128 = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128);
  // Measured on MI355X (fp16, 256 CUs, every epilogue).
  // Whole 256x256 tiles (the ping-pong loop has no row clamp and runs K-tiles
  // in pairs) that fill at least one round of the CUs take the ping-pong loop,
  // short K included: C4 forward 9.07 -> 8.62 ms, every 256x256 GEMM role 6-9 %
  // faster than the two-stage loop; C3 out-projection (one round, K = 1024)
  // 62.0 -> 54.4 us against the 128x128 tile; C2 FFN-up (two rounds, K = 512)
  // unchanged.
  // (its epilogues also assume vector-aligned output rows and bias).
  if (t256 >= 256 && p.M % 256 == 0 && p.N % 256 == 0 && p.K > 0 && p.K % 128 == 0 && p.vec &&
      (p.bias == nullptr || p.bias16)) {
    if constexpr (EPI == TK_EPI_BIAS || EPI == TK_EPI_BIAS_GELU || EPI == TK_EPI_BIAS_RESID) {
      if (kGemmPf && p.kvec && t256 > kPfGrid) {  // some workgroup runs two or more tiles
        hipLaunchKernelGGL((gemm_pf_kernel<TileBigPP, EPI>), dim3((unsigned)kPfGrid), dim3(TileBigPP::NT), 0, st, p);
        return check_launch("tk_gemm");
      }
    }
    return launch_gemm<TileBigPP, EPI>(p, st);
  }
  // Other shapes, with the two-stage loop: 256x256 tiles win when they fill
  // whole rounds of the 256 CUs (or at least two rounds); with a partial last
  // round (e.g. 384 tiles) the 128x128 tile, two blocks per CU, is 5-10 %
  // faster, as it is for narrow and short outputs down to 128 of its tiles;
  // below that the 64x64 tile keeps the CUs busy.  Short K (<= 1024) with at
  // most two rounds of 256x256 tiles also runs 128x128 tiles (0.5-4 % faster);
  // larger K or more rounds favour 256x256.
  const bool short_k = p.K <= 1024 && t256 <= 512;
  if (!short_k && t256 >= 256 && (t256 % 256 == 0 || t256 >= 512)) return launch_gemm<TileBig, EPI>(p, st);
  if (t128 >= 128) return launch_gemm<TileMid, EPI>(p, st);
  return launch_gemm<TileSmall, EPI>(p, st);
}

template <class T>
int launch_gemm_ln(const GemmArgs& p, bool h_half, hipStream_t st) {
  const dim3 grid((unsigned)((p.M + T::BM - 1) / T::BM)), block(T::NT);
  if (p.K % T::BK == 0 && p.kvec) {
    if (h_half) hipLaunchKernelGGL((gemm_ln_kernel<T, true, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((gemm_ln_kernel<T, false, true>), grid, block, 0, st, p);
  } else {
    if (h_half) hipLaunchKernelGGL((gemm_ln_kernel<T, true, false>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((gemm_ln_kernel<T, false, false>), grid, block, 0, st, p);
  }
  return check_launch("tk_gemm_bias_add_ln");
}

// ---- fused QKV projection + one-tile attention (S = 64, head_dim = 64) ----
// One workgroup computes, for 128 tokens (two sequences) and one head h, the
// 128 x 192 tile [Q_h | K_h | V_h] = h . [Wq_h | Wk_h | Wv_h]^T + b (fp32
// accumulate, bias in fp32, fp16 rounding -- the values the plain QKV GEMM
// would store), stages it in LDS in the single-tile attention layouts and
// runs that attention for both sequences (waves 2s, 2s+1: query rows 0-31
// and 32-63 of sequence s).  Q, K and V never reach HBM; only the context
// [tokens, d_model] is written.  Results are those of the QKV GEMM followed
// by the single-tile flash kernel.
constexpr int kQaHD = 64;                 // head_dim
constexpr int kQaS = 64;                  // sequence length (one key tile)
constexpr int kQaRows = 128;              // tokens per workgroup
constexpr int kQaTile = kQaS * kQaHD * 2; // bytes of one K or V tile
using QaLoop = Mainloop<kQaRows, 3 * kQaHD, 2, 2, 64, 2, true, kQaHD>;

struct QaArgs {
  f16* ctx;
  int64_t ldo;
  int H;
  float scale_log2;
};

template <bool CAUSAL>
__global__ __launch_bounds__(256, 2) void qkv_attn_kernel(GemmArgs p, QaArgs a) {
  static_assert(QaLoop::FM == 2 && QaLoop::FN == 3 && QaLoop::NW == 4, "4 waves of 64 x 96");
  __shared__ __attribute__((aligned(16))) f16 smem[QaLoop::LDS_HALVES];
  static_assert(QaLoop::LDS_HALVES * 2 >= kQaRows * kQaHD * 2 + 4 * kQaTile, "Q, K and V staging fits");
  const int tiles_m = p.M / kQaRows;
  int tm, h;
  tile_of_block(blockIdx.x, tiles_m, a.H, tm, h);
  const int m0 = tm * kQaRows;
  f32x16 acc[QaLoop::FN][QaLoop::FM];
  QaLoop::run(p, m0, h * kQaHD, smem, acc);

  char* lds = reinterpret_cast<char*>(smem);
  char* q_s = lds;                                 // [128 rows][128 B], chunk-swizzled
  char* k_s = lds + kQaRows * kQaHD * 2;           // two K tiles
  char* v_s = k_s + 2 * kQaTile;                   // two V tiles
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave % 2, wn = wave / 2;
  const int g = lane >> 5;
  __syncthreads();  // every wave is done with the main-loop buffers
  // accumulator element (i, j, 4q+e): row wm*64 + 32j + (lane & 31),
  // column wn*96 + 32i + 8q + 4g + e of [Q | K | V]
#pragma unroll
  for (int i = 0; i < QaLoop::FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = wn * 96 + i * 32 + 8 * q + 4 * g;
      const int part = n / kQaHD, d = n % kQaHD;  // 0 Q, 1 K, 2 V
      const f32x4 bv = *reinterpret_cast<const f32x4*>(p.bias + (int64_t)part * p.w_gstride + h * kQaHD + d);
#pragma unroll
      for (int j = 0; j < QaLoop::FM; ++j) {
        const int m = wm * 64 + j * 32 + (lane & 31);
        const f16x4 t = {(f16)(acc[i][j][4 * q] + bv[0]), (f16)(acc[i][j][4 * q + 1] + bv[1]),
                         (f16)(acc[i][j][4 * q + 2] + bv[2]), (f16)(acc[i][j][4 * q + 3] + bv[3])};
        const int sq = m / kQaS, r = m % kQaS;
        char* dst;
        if (part == 0) dst = q_s + swz_off<2 * kQaHD>(m, d >> 3) + (d & 7) * 2;
        else if (part == 1) dst = k_s + sq * kQaTile + swz_off<2 * kQaHD>(r, d >> 3) + (d & 7) * 2;
        else dst = v_s + sq * kQaTile + r * (2 * kQaHD) + (((d >> 3) ^ vswz<2 * kQaHD>(r)) << 4) + (d & 7) * 2;
        *reinterpret_cast<f16x4*>(dst) = t;
      }
    }
  __syncthreads();

  const int sq = wave / 2;                      // sequence of this wave
  const int my_row = (wave % 2) * 32 + (lane & 31);
  f16x8 qf[kQaHD / 16];
#pragma unroll
  for (int kk = 0; kk < kQaHD / 16; ++kk)
    qf[kk] = *reinterpret_cast<const f16x8*>(q_s + swz_off<2 * kQaHD>(sq * kQaS + my_row, 2 * kk + g));
  attend_one_tile<kQaHD, CAUSAL, false>(k_s + sq * kQaTile, v_s + sq * kQaTile, qf, my_row, kQaS, 0ull,
                                        a.scale_log2, a.ctx + (int64_t)(m0 + sq * kQaS) * a.ldo + h * kQaHD,
                                        a.ldo);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace
}  // namespace tk

using namespace tk;

extern "C" int tk_gemm(const tk_half* a, int64_t lda, const tk_half* w, int64_t ldw,
                       const float* bias, const float* resid, int64_t ldr, void* c, int64_t ldc,
                       int64_t m, int64_t n, int64_t k, int epilogue, const uint8_t* row_valid,
                       int row_mode, void* stream) {
  TK_REQUIRE(a && w && c, TK_ERR_ARG, "tk_gemm: null pointer");
  TK_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31),
             TK_ERR_ARG, "tk_gemm: bad sizes m=%lld n=%lld k=%lld", (long long)m, (long long)n,
             (long long)k);
  TK_REQUIRE(lda >= k && ldw >= k, TK_ERR_ARG, "tk_gemm: lda=%lld ldw=%lld must be >= k=%lld",
             (long long)lda, (long long)ldw, (long long)k);
  TK_REQUIRE(((uintptr_t)a & 1) == 0 && ((uintptr_t)w & 1) == 0, TK_ERR_ARG,
             "tk_gemm: A and W must be 2-byte aligned");
  TK_REQUIRE(epilogue == TK_EPI_BIAS || epilogue == TK_EPI_BIAS_GELU || epilogue == TK_EPI_BIAS_RESID,
             TK_ERR_ARG, "tk_gemm: bad epilogue %d", epilogue);
  TK_REQUIRE(ldc >= n, TK_ERR_ARG, "tk_gemm: ldc=%lld < n=%lld", (long long)ldc, (long long)n);
  if (epilogue == TK_EPI_BIAS_RESID)
    TK_REQUIRE(resid != nullptr && ldr >= n, TK_ERR_ARG, "tk_gemm: residual epilogue needs resid, ldr >= n");
  TK_REQUIRE(row_valid == nullptr || (epilogue == TK_EPI_BIAS_RESID && row_mode >= TK_ROWS_KEEP_RESID &&
                                      row_mode <= TK_ROWS_ZERO_ALL),
             TK_ERR_ARG, "tk_gemm: row_valid needs the residual epilogue and a tk_row_mode (got %d)", row_mode);
  if (m == 0 || n == 0) return TK_OK;
  GemmArgs p{};
  p.row_valid = row_valid;
  p.row_mode = row_mode;
  // 16-byte vector stores (and residual loads) when every output row start
  // is aligned for them; element-wise otherwise.
  if (epilogue == TK_EPI_BIAS_RESID)
    p.vec = aligned16(resid) && aligned16(c) && ldr % 4 == 0 && ldc % 4 == 0;
  else
    p.vec = aligned16(c) && ldc % 8 == 0;
  p.bias16 = bias != nullptr && aligned16(bias);
  p.kvec = k % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0 && aligned16(a) && aligned16(w);
  p.a = reinterpret_cast<const f16*>(a);
  p.w = reinterpret_cast<const f16*>(w);
  p.bias = bias;
  p.resid = resid;
  p.c = c;
  p.lda = lda; p.ldw = ldw; p.ldr = ldr; p.ldc = ldc;
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  hipStream_t st = as_stream(stream);
  switch (epilogue) {
    case TK_EPI_BIAS: return gemm_dispatch<TK_EPI_BIAS>(p, st);
    case TK_EPI_BIAS_GELU: return gemm_dispatch<TK_EPI_BIAS_GELU>(p, st);
    default:
      return p.row_valid ? gemm_dispatch<kEpiResidRows>(p, st) : gemm_dispatch<TK_EPI_BIAS_RESID>(p, st);
  }
}

extern "C" int tk_gemm_ln_supported(int64_t n) { return n == 128 || n == 256 || n == 512; }

extern "C" int tk_gemm_bias_add_ln(const tk_half* a, int64_t lda, const tk_half* w, int64_t ldw,
                                   const float* bias, const float* resid, const float* ln_w,
                                   const float* ln_b, float* sum_out, void* h_out, int h_dtype,
                                   int64_t m, int64_t n, int64_t k, float eps, const uint8_t* row_valid,
                                   int row_mode, void* stream) {
  TK_REQUIRE(a && w && resid && ln_w && ln_b && h_out, TK_ERR_ARG, "tk_gemm_bias_add_ln: null pointer");
  TK_REQUIRE(tk_gemm_ln_supported(n), TK_ERR_UNSUPPORTED,
             "tk_gemm_bias_add_ln: row width n=%lld not in {128, 256, 512}", (long long)n);
  TK_REQUIRE(m >= 0 && m < (1ll << 31) && k >= 0 && k < (1ll << 31), TK_ERR_ARG,
             "tk_gemm_bias_add_ln: bad sizes");
  TK_REQUIRE(lda >= k && ldw >= k, TK_ERR_ARG, "tk_gemm_bias_add_ln: lda, ldw must be >= k");
  TK_REQUIRE(h_dtype == TK_F16 || h_dtype == TK_F32, TK_ERR_ARG, "tk_gemm_bias_add_ln: bad h_dtype");
  TK_REQUIRE(((uintptr_t)a & 1) == 0 && ((uintptr_t)w & 1) == 0 && aligned16(resid) && aligned16(ln_w) &&
                 aligned16(ln_b) &&
                 aligned16(h_out) && (sum_out == nullptr || aligned16(sum_out)) &&
                 (bias == nullptr || aligned16(bias)),
             TK_ERR_ARG, "tk_gemm_bias_add_ln: buffers must be 16-byte aligned");
  TK_REQUIRE(row_valid == nullptr || (row_mode >= TK_ROWS_KEEP_RESID && row_mode <= TK_ROWS_ZERO_ALL),
             TK_ERR_ARG, "tk_gemm_bias_add_ln: bad row_mode %d", row_mode);
  if (m == 0) return TK_OK;
  GemmArgs p{};
  p.row_valid = row_valid;
  p.row_mode = row_mode;
  p.a = reinterpret_cast<const f16*>(a);
  p.w = reinterpret_cast<const f16*>(w);
  p.bias = bias;
  p.resid = resid;
  p.c = h_out;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.sum_out = sum_out;
  p.kvec = k % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0 && aligned16(a) && aligned16(w);
  p.lda = lda; p.ldw = ldw; p.ldr = n; p.ldc = n;
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  p.eps = eps;
  hipStream_t st = as_stream(stream);
  const bool hh = h_dtype == TK_F16;
  if (n == 512) return launch_gemm_ln<Tile<64, 512, 1, 8, 64, 2>>(p, hh, st);
  if (n == 256) return launch_gemm_ln<Tile<64, 256, 1, 4, 64, 2>>(p, hh, st);
  return launch_gemm_ln<Tile<64, 128, 1, 2, 64, 2>>(p, hh, st);
}

extern "C" int tk_qkv_attention_supported(int64_t batch, int64_t seq, int64_t heads, int64_t head_dim) {
  return seq == kQaS && head_dim == kQaHD && heads >= 1 && batch >= 0 && (batch * seq) % kQaRows == 0;
}

extern "C" int tk_qkv_attention(const tk_half* h, int64_t ldh, const tk_half* w_qkv, int64_t ldw,
                                const float* b_qkv, tk_half* ctx, int64_t ldc, int64_t batch, int64_t seq,
                                int64_t heads, int64_t head_dim, float scale, int causal, void* stream) {
  TK_REQUIRE(h && w_qkv && b_qkv && ctx, TK_ERR_ARG, "tk_qkv_attention: null pointer");
  TK_REQUIRE(tk_qkv_attention_supported(batch, seq, heads, head_dim), TK_ERR_UNSUPPORTED,
             "tk_qkv_attention: needs seq=%d, head_dim=%d and batch*seq a multiple of %d (got batch=%lld "
             "seq=%lld head_dim=%lld)",
             kQaS, kQaHD, kQaRows, (long long)batch, (long long)seq, (long long)head_dim);
  const int64_t d = heads * head_dim;
  TK_REQUIRE(d < (1 << 20) && batch * seq < (1ll << 31), TK_ERR_ARG, "tk_qkv_attention: bad sizes");
  TK_REQUIRE(ldh >= d && ldh % 8 == 0 && ldw >= d && ldw % 8 == 0 && ldc >= d && ldc % 4 == 0, TK_ERR_ARG,
             "tk_qkv_attention: ldh, ldw must be multiples of 8 and ldc of 4, each >= d_model");
  TK_REQUIRE(aligned16(h) && aligned16(w_qkv) && aligned16(b_qkv) && ((uintptr_t)ctx & 7) == 0, TK_ERR_ARG,
             "tk_qkv_attention: h, w_qkv, b_qkv need 16-byte and ctx 8-byte alignment");
  if (batch == 0) return TK_OK;
  GemmArgs p{};
  p.a = reinterpret_cast<const f16*>(h);
  p.w = reinterpret_cast<const f16*>(w_qkv);
  p.bias = b_qkv;
  p.lda = ldh;
  p.ldw = ldw;
  p.M = (int)(batch * seq);
  p.N = (int)(3 * d);
  p.K = (int)d;
  p.w_gstride = d;
  QaArgs qa{reinterpret_cast<f16*>(ctx), ldc, (int)heads, scale * 1.4426950408889634f};
  const dim3 grid((unsigned)((int64_t)(p.M / kQaRows) * heads)), block(256);
  if (causal) hipLaunchKernelGGL((qkv_attn_kernel<true>), grid, block, 0, as_stream(stream), p, qa);
  else hipLaunchKernelGGL((qkv_attn_kernel<false>), grid, block, 0, as_stream(stream), p, qa);
  return check_launch("tk_qkv_attention");
}
