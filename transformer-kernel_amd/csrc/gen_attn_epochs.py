"""Emit tk_attn_epochs.inc and tk_attn_epochs_kmask.inc: the hand-ordered steady-state epochs of
the head_dim-128 causal attention (flash_pair_body in tk_attention.hip, 8 waves, 256 query rows
per workgroup), without and with a key mask.

    python gen_attn_epochs.py [outdir]      # default: beside this file

The build runs this before compiling tk_attention.hip, so the .inc files and this script cannot
drift.

What an epoch computes
----------------------
Epoch e of the pair body (key tile e = keys 64e .. 64e+63) does, for every wave:

  copies    K tile e+2 into K slot (e+2) % 3, V tile e+1 into V slot (e+1) % 4 (LDS DMA)
  S phase   S^T(e) = K(e) . Q^T, 16 MFMAs 32x32x16; MFMA c: key block c & 1, k-step c >> 1
  max       m_tile = scale*log2(e) * max over the lane pair; lazy rescale when any lane's
            m_tile exceeds m_run + 8: m_new = max(m_run, m_tile), alpha = exp2(m_run - m_new),
            l_run *= alpha
  P.V phase O^T += V^T(e-1) . P^T(e-1), 16 MFMAs (head-dim block c & 3, P block c >> 2),
            with P(e) = fp16(exp2(s * cs - m_run)) and its fp16 row sum (dot2 with 1.0h)
            computed between them
  rescale   O *= alpha when the rescale ran
  end       wait for the previous epoch's copies, barrier

Each lane computes every value the compiled epoch keeps (P, m, l, O) with the same operations on
the same operands in the same order, so the results are bit-identical to it (the dense loop
computes the row max only when it can matter, below).  The loop covers the epochs [1, 1 + 4*groups),
which the host side chooses so that no key tile in them needs a causal or length mask (every key
is below every query row of the workgroup) and no copy is clamped to the last tile.  Without a
key mask m_run is finite there (epoch 0 saw key 0).  With one, every row of the workgroup has
seen the same keys with the same validity (no causal mask applies in these epochs), so m_run and
m_tile are -inf for all rows of a wave or for none: the wave-wide rescale test never fires for a
row whose m_new would be -inf.  The rescale still maps m_new = -inf to alpha = 1 (one compare and
one select on that rare path), so l and O cannot turn into NaN if the loop's gate ever admits
rows with different key histories.

The key-masked loop (one_phase_program) runs each epoch in that order.  The dense loop
(program_spread) computes the same values per lane, but software-pipelined so that every one of
an iteration's 32 MFMA slots carries a share of the softmax: iteration e runs the P.V MFMAs of
epoch e (slots 0..15) and the score MFMAs of epoch e+1 (key block 0 in slots 16..23, key block 1
in 24..31); between them the 16 exponential pairs of S(e), computed in place on the score
registers (slots 1..23), and the row sums in pair order (24..31).  It skips the row max: the
exponentials use m_run as it stands, which is what the compiled epoch does whenever its lazy
rescale does not fire (m_tile <= m_run + 8 on every lane).  When it fires, some P entry is
exp2(m_tile - m_run) > 2^8 against m_run, so that lane's row sum is at least 256; a row sum of
128 or more on any lane (or inf / NaN) therefore sends the wave to the iteration's refit block,
which recomputes S(e), takes its row max and applies the compiled epoch's rescale test and
update, and recomputes P(e), its row sums and S(e+1) -- the outputs stay bit-identical to the
compiled epochs, and the row max costs nothing while no row max moves by more than a few
units (C4: 1070-1072 -> 1037-1038 us against the loop with the max in slots 0..2, same box).  The scores of epoch 1
are computed before the loop; the last iteration also computes the scores of the epoch after the
loop, which the compiled epoch recomputes (16 MFMAs per loop).  Two waves of a SIMD issuing
MFMAs with at most about three VALU instructions and one exponential between each pair run at
the MFMA rate; the one-phase epoch, with its 32 exponentials between 16 of its MFMAs and none
between the other 16, cannot hide them.

One loop iteration is 4 epochs, so epoch e = 1 + 4i + u (loop position u) reads V(e-1) from
V slot (e-1) % 4 = u and writes V(e+1) into slot (u + 2) % 4: both are immediate LDS offsets.
The K ring has 3 slots, so its read and write slots rotate through the SGPR trackers krd and kwr
(byte offsets of the slots, starting at slots 1 and 0 for epoch 1).  The dense loop reads K(e+1)
in iteration e, so it waits at the end of iteration e for the K copy of that iteration
(vmcnt(2): the V copies, issued after it, may stay in flight) and advances krd once after the
scores of epoch 1.  It copies V two epochs ahead (V(e+2) into V slot (e+2) % 4, which held
V(e-2); V(2) before the loop), so V(e) has landed and passed a barrier by the end of iteration
e, whose last two slots already read the first two V(e) fragments of the next iteration.

Register map (all VGPRs; the asm statement pins or clobbers every one of them)
-------------------------------------------------------------------------------
  v[64:127]   O^T accumulators, 4 x 16          (in/out)
  v[128:159]  Q fragments, 8 x 4                 (in)
  v[160:175]  P tile region A                     (in/out: holds P(e-1) at entry and exit)
  v[176:191]  P tile region B                     (clobbered)
  v192, v193  m_run, l_run                        (in/out)
  v194..v197  T0, T1, ALPHA, LS (row-sum partial) (clobbered); MX = T0 and TMP = T1 (the S and
              max phases use MX/TMP, the P.V phase T0/T1; the dense loop uses them, and
              ALPHA, only in its refit blocks)
  v[198:213]  scores, key block 1                 (clobbered)
  v[214:225]  operand ring, 3 x 4: K fragments in the S phase, V fragments in the P.V phase
  v[226:227]  second temporary pair of the exponential pipeline (clobbered); in the dense loop
              the K read address and its base (krd + kl0)
Scores of key block 0 live in the region that receives the new P tile: P.V step c writes P
register c after reading scores 2c and 2c+1, and score c was read at step c // 2.  Regions A and
B alternate between "P being consumed" and "scores block 0 / new P" from epoch to epoch.  The
dense loop exponentiates in place (score register -> scaled -> exp2 -> packed into P register j),
so it needs no temporary pairs; its score MFMAs of epoch e+1 write key block 0 into the region P
of epoch e-1 leaves (after the P.V MFMAs that read it) and key block 1 into v[198:213] (after
the last exponential pair of epoch e has read it).

Wait states given for the hazards the hardware does not interlock (each at least what the
compiler inserts for gfx950 in the same situation)
------------------------------------------------------------------------------------------
  SALU write of M0 -> LDS DMA reading M0                1   (s_nop 0)
  MFMA 32x32 result -> VALU read or write               24  (3 x s_nop 7)
  VALU write       -> v_permlane32_swap read            2   (s_nop 1)
  VALU write VCC   -> s_cbranch_vccz                    4   (s_nop 3)
  v_exp (trans.)   -> non-trans. VALU read              1   (s_nop 0)
  v_dot2c result   -> different VALU read               3   (s_nop 2)
  MFMA accumulate chains and same-opcode v_dot2c accumulate chains need none.
"""
from __future__ import annotations

import pathlib
import sys

O = 64                # v[64:127]  O^T accumulators, 4 x 16
Q = 128               # v[128:159] Q fragments, 8 x 4
P = (160, 176)        # the two 16-register P regions
MR, LR = 192, 193     # m_run, l_run
T0, T1, ALPHA, LS = 194, 195, 196, 197
MX, TMP = T0, T1
SB1 = 198             # v[198:213] scores, key block 1
RING = 214            # v[214:225] K (S phase) / V (P.V phase) fragment ring
TX = 226              # v[226:227] a second exponential pair in flight (P.V phase)
TILE = 16384          # bytes per K or V tile in LDS (64 rows x 256 bytes)

PINNED = set(range(64, 176)) | {MR, LR}               # operands of the asm statement
CLOBBERED = sorted(set(range(176, 192)) | set(range(194, 228)))


def v(a: int, n: int = 1) -> str:
    return f"v{a}" if n == 1 else f"v[{a}:{a + n - 1}]"


# key-masked variant: physical SGPRs (inline asm cannot name halves of a 64-bit operand)
S_MASK = (88, 90)     # two lane-mask pairs, alternating
S_KB = (92, 93)       # key-validity bits of the tile: lanes' keys 0..31, 32..63
S_NOKEY = 94          # s[94:95]: lanes whose m_run is still -inf (no valid key yet)
S_CLOBBERED = list(range(88, 96))
NEG_INF = "0xff800000"
P_CHECK = "0x43000000"  # 128.0f: the row-sum level that sends a wave to the exact row max


def key_mask(sr, neg: int = ALPHA) -> list[str]:
    """Scores of keys whose validity byte is 0 -> -inf (held in register `neg`).  Entry
    i = 16*kb2 + r of a lane holds key 32*kb2 + 8*(r/4) + r%4 + 4g (g = lane / 32), so its lane
    mask takes bit j of the tile's bits (s92: keys 0..31, s93: 32..63) for lanes 0..31 and bit
    j+4 for lanes 32..63 (s_bfe_i32 of one bit: 0 or -1)."""
    def mask(i: int, pair: int) -> list[str]:
        kb2, r = i >> 4, i & 15
        j = 32 * kb2 + 8 * (r >> 2) + (r & 3)
        lo, hi = j, j + 4
        return [f"s_bfe_i32 s{pair}, s{S_KB[lo >> 5]}, {(lo & 31) | (1 << 16)}",
                f"s_bfe_i32 s{pair + 1}, s{S_KB[hi >> 5]}, {(hi & 31) | (1 << 16)}"]

    def select(i: int, pair: int) -> list[str]:
        return [f"v_cndmask_b32 {v(sr(i))}, {v(neg)}, {v(sr(i))}, s[{pair}:{pair + 1}]"]

    out = [f"v_mov_b32 {v(neg)}, {NEG_INF}"] + mask(0, S_MASK[0])
    for i in range(32):
        if i + 1 < 32:
            out += mask(i + 1, S_MASK[(i + 1) % 2])  # two instructions between a mask and its use
        out += select(i, S_MASK[i % 2])
    return out


def epoch(u: int, kmask: bool = False) -> list[str]:
    """Instructions of the epoch at loop position u (0..3); kmask: the key-masked variant."""
    pp, pc = (P[0], P[1]) if u % 2 == 0 else (P[1], P[0])
    sb = (pc, SB1)  # scores: key block 0 in the new-P region, key block 1 in SB1

    def sr(i: int) -> int:  # register of score i (0..31) = accumulator entry i & 15 of block i >> 4
        return sb[i >> 4] + (i & 15)

    L = ["s_mov_b32 %[flag], 0", f"v_mov_b32 {v(LS)}, 0"]
    if kmask:  # this tile's key-validity bytes, one per lane, ahead of the copies (vmcnt order)
        L += [f"global_load_ubyte {v(TX)}, %[koff], %[kvb]", "v_add_u32 %[koff], 64, %[koff]"]
    # ---- copies: K(e+2) into the K slot kwr, V(e+1) into V slot (u + 2) % 4 ----
    L += ["s_add_u32 m0, %[ldsw], %[kwr]", "s_nop 0", "global_load_lds_dwordx4 %[ko0], %[kb]",
          "s_add_u32 m0, m0, 8192", "s_nop 0", "global_load_lds_dwordx4 %[ko1], %[kb]"]
    vw = (3 + (u + 2) % 4) * TILE
    L += [f"s_add_u32 m0, %[ldsw], {vw}", "s_nop 0", "global_load_lds_dwordx4 %[vo0], %[vb]",
          f"s_add_u32 m0, %[ldsw], {vw + 8192}", "s_nop 0", "global_load_lds_dwordx4 %[vo1], %[vb]"]
    L += ["v_add_u32 %[ko0], %[kt2], %[ko0]", "v_add_u32 %[ko1], %[kt2], %[ko1]",
          "v_add_u32 %[vo0], %[vt2], %[vo0]", "v_add_u32 %[vo1], %[vt2], %[vo1]"]

    # ---- S phase: fragment reads run two MFMAs ahead through the 3-entry ring ----
    def kread(c: int) -> list[str]:
        # k-step kk reads chunk 2kk + g of the XOR-swizzled row: row offset kl0 ^ (kk << 5)
        out = []
        if c % 2 == 0:
            kk = c >> 1
            if kk == 0:
                out.append(f"v_add_u32 {v(TMP)}, %[krd], %[kl0]")
            else:
                out += [f"v_xor_b32 {v(TMP)}, {kk << 5}, %[kl0]", f"v_add_u32 {v(TMP)}, %[krd], {v(TMP)}"]
        out.append(f"ds_read_b128 {v(RING + 4 * (c % 3), 4)}, {v(TMP)} offset:{(c & 1) * 8192}")
        return out

    L += kread(0) + kread(1)
    for c in range(16):
        if c + 2 < 16:
            L += kread(c + 2)
        L.append(f"s_waitcnt lgkmcnt({min(2, 15 - c)})")
        src_c = "0" if (c >> 1) == 0 else v(sb[c & 1], 16)
        L.append(f"v_mfma_f32_32x32x16_f16 {v(sb[c & 1], 16)}, {v(RING + 4 * (c % 3), 4)}, "
                 f"{v(Q + 4 * (c >> 1), 4)}, {src_c}")

    # ---- row max over the lane pair, lazy rescale ----
    # two interleaved chains (key blocks 0 and 1), so no max waits on the one before it
    L += ["s_nop 7", "s_nop 7", "s_nop 7"]
    if kmask:  # the byte load is older than this epoch's four copies
        L += ["s_waitcnt vmcnt(4)", f"v_cmp_ne_u32 vcc, 0, {v(TX)}",
              f"s_mov_b32 s{S_KB[0]}, vcc_lo", f"s_mov_b32 s{S_KB[1]}, vcc_hi"]
        L += key_mask(sr)
    L += [f"v_max3_f32 {v(MX)}, {v(sr(0))}, {v(sr(1))}, {v(sr(2))}",
          f"v_max3_f32 {v(TMP)}, {v(sr(16))}, {v(sr(17))}, {v(sr(18))}"]
    for k in range(3, 15, 2):
        L += [f"v_max3_f32 {v(MX)}, {v(MX)}, {v(sr(k))}, {v(sr(k + 1))}",
              f"v_max3_f32 {v(TMP)}, {v(TMP)}, {v(sr(16 + k))}, {v(sr(17 + k))}"]
    L += [f"v_max3_f32 {v(MX)}, {v(MX)}, {v(sr(15))}, {v(TMP)}",
          f"v_max_f32 {v(MX)}, {v(MX)}, {v(sr(31))}"]
    L += [f"v_mov_b32 {v(TMP)}, {v(MX)}", "s_nop 1", f"v_permlane32_swap_b32 {v(MX)}, {v(TMP)}",
          f"v_max_f32 {v(MX)}, {v(MX)}, {v(TMP)}",
          f"v_mul_f32 {v(MX)}, %[cs], {v(MX)}",                 # m_tile
          f"v_add_f32 {v(TMP)}, 0x41000000, {v(MR)}",            # m_run + 8
          f"v_cmp_gt_f32 vcc, {v(MX)}, {v(TMP)}", "s_nop 3",
          f"s_cbranch_vccz L_norescale_{u}_%="]
    L += [f"v_max_f32 {v(TMP)}, {v(MR)}, {v(MX)}",               # m_new
          f"v_sub_f32 {v(ALPHA)}, {v(MR)}, {v(TMP)}",
          f"v_exp_f32 {v(ALPHA)}, {v(ALPHA)}",
          f"v_cmp_eq_f32 vcc, {NEG_INF}, {v(TMP)}",              # m_new = -inf: alpha = 1
          f"v_mov_b32 {v(MR)}, {v(TMP)}",
          f"v_cndmask_b32 {v(ALPHA)}, {v(ALPHA)}, 1.0, vcc",
          f"v_mul_f32 {v(LR)}, {v(LR)}, {v(ALPHA)}",
          "s_mov_b32 %[flag], 1"]
    L += [f"L_norescale_{u}_%=:"]
    if kmask:  # rows with no valid key so far: exponentials against 0, m_run restored after
        L += [f"v_cmp_eq_f32 vcc, {NEG_INF}, {v(MR)}", f"s_mov_b64 s[{S_NOKEY}:{S_NOKEY + 1}], vcc",
              f"v_cndmask_b32 {v(MR)}, {v(MR)}, 0, vcc"]

    # ---- P.V phase: O^T += V^T(e-1) P^T(e-1); exponentials of S(e) between the MFMAs ----
    vslot = u * TILE

    def vread(c: int) -> list[str]:
        t, d = c >> 2, c & 3
        base = RING + 4 * (c % 3)
        # the second half-fragment sits 8 tile rows (2048 bytes) further, same swizzle
        return [f"ds_read_b64_tr_b16 {v(base, 2)}, %[vl{d}] offset:{vslot + t * 4096}",
                f"ds_read_b64_tr_b16 {v(base + 2, 2)}, %[vl{d}] offset:{vslot + t * 4096 + 2048}"]

    # Exponential pair j (scores 2j, 2j+1 -> P register j) runs as a two-stage pipeline
    # over the MFMA slots: scaled at slot j-1, then at slot j exponentiated, the next pair
    # scaled, and packed and summed -- the two scalings sit between each exponential and its
    # pack.  Two temporary pairs alternate; the row sum still adds pairs in order 0..15.
    tpair = ((T0, T1), (TX, TX + 1))

    def scale(j: int) -> list[str]:
        a, b = tpair[j % 2]
        return [f"v_fma_f32 {v(a)}, {v(sr(2 * j))}, %[cs], -{v(MR)}",
                f"v_fma_f32 {v(b)}, {v(sr(2 * j + 1))}, %[cs], -{v(MR)}"]

    def expo(j: int) -> list[str]:
        a, b = tpair[j % 2]
        return [f"v_exp_f32 {v(a)}, {v(a)}", f"v_exp_f32 {v(b)}, {v(b)}"]

    def pack(j: int) -> list[str]:
        a, b = tpair[j % 2]
        return [f"v_cvt_pk_f16_f32 {v(pc + j)}, {v(a)}, {v(b)}",
                f"v_dot2c_f32_f16 {v(LS)}, 0x3c003c00, {v(pc + j)}"]

    L += vread(0) + vread(1) + scale(0)
    for c in range(16):
        if c + 2 < 16:
            L += vread(c + 2)
        L.append(f"s_waitcnt lgkmcnt({2 * min(2, 15 - c)})")
        L.append(f"v_mfma_f32_32x32x16_f16 {v(O + 16 * (c & 3), 16)}, {v(RING + 4 * (c % 3), 4)}, "
                 f"{v(pp + 4 * (c >> 2), 4)}, {v(O + 16 * (c & 3), 16)}")
        L += expo(c)
        L += scale(c + 1) if c + 1 < 16 else ["s_nop 1"]
        L += pack(c)
    L += ["s_nop 2", f"v_add_f32 {v(LR)}, {v(LR)}, {v(LS)}"]
    # ---- O rescale ----
    L += ["s_cmp_eq_u32 %[flag], 0", f"s_cbranch_scc1 L_noscale_{u}_%=", "s_nop 7", "s_nop 7", "s_nop 7"]
    L += [f"v_mul_f32 {v(O + r)}, {v(O + r)}, {v(ALPHA)}" for r in range(64)]
    L += [f"L_noscale_{u}_%=:"]
    if kmask:
        L += [f"v_mov_b32 {v(ALPHA)}, {NEG_INF}",
              f"v_cndmask_b32 {v(MR)}, {v(MR)}, {v(ALPHA)}, s[{S_NOKEY}:{S_NOKEY + 1}]"]
    # ---- end: this epoch's copies may stay in flight, the previous epoch's have landed ----
    L += ["s_waitcnt vmcnt(4)", "s_barrier",
          "s_add_u32 %[krd], %[krd], 16384", "s_cmp_eq_u32 %[krd], 49152", "s_cselect_b32 %[krd], 0, %[krd]",
          "s_add_u32 %[kwr], %[kwr], 16384", "s_cmp_eq_u32 %[kwr], 49152", "s_cselect_b32 %[kwr], 0, %[kwr]"]
    return L


# --------------------------------------------------------------------------- #
# the dense loop: softmax work spread over all 32 MFMA slots of an iteration
# --------------------------------------------------------------------------- #
# Relative VALU issue cost of one instruction (cycles of a lone wave): exponentials occupy the
# transcendental unit about 8.6 cycles, the rest about 5.3.  Used only to spread the work evenly.
def _cost(ins: str) -> float:
    return 8.6 if ins.startswith("v_exp") else 5.3 if ins.startswith("v_") else 1.0


def _spread(ops: list[str], slots: list[list[str]], first: int, last: int) -> None:
    """Append the instructions, in order, to slots first..last, cutting the stream by issue cost."""
    total = sum(_cost(i) for i in ops)
    n, acc = last - first + 1, 0.0
    for i in ops:
        slots[min(first + int((acc + _cost(i) / 2) * n / total), last)].append(i)
        acc += _cost(i)


def block0_max(x: int) -> list[str]:
    """MX = max of the key-block-0 scores (accumulator entries x .. x+15)."""
    L = [f"v_max3_f32 {v(MX)}, {v(x)}, {v(x + 1)}, {v(x + 2)}"]
    L += [f"v_max3_f32 {v(MX)}, {v(MX)}, {v(x + k)}, {v(x + k + 1)}" for k in range(3, 15, 2)]
    return L + [f"v_max_f32 {v(MX)}, {v(MX)}, {v(x + 15)}"]


def vread(c: int, u: int) -> list[str]:
    """V fragment c of the P.V MFMAs at loop position u (V slot u) into ring entry c % 3; the
    second half-fragment sits 8 tile rows (2048 bytes) further, same swizzle."""
    t, d, base = c >> 2, c & 3, RING + 4 * (c % 3)
    return [f"ds_read_b64_tr_b16 {v(base, 2)}, %[vl{d}] offset:{u * TILE + t * 4096}",
            f"ds_read_b64_tr_b16 {v(base + 2, 2)}, %[vl{d}] offset:{u * TILE + t * 4096 + 2048}"]


def spread_iteration(u: int) -> list[str]:
    """Iteration at loop position u (epoch e = 1 + 4i + u) of the dense loop.

    MFMA slots 0..15: O^T += V^T(e-1) P^T(e-1) (head-dim block c & 3, P block c >> 2);
    slots 16..23: S^T(e+1) key block 0 (k-steps 0..7), slots 24..31: key block 1 (k-steps 0..7).
    VALU work between them: the 16 exponential pairs of S(e) against the running reference
    m_run (no row max), each computed in place on its two score registers and packed into P
    register j (slots 1..23: the pairs of key block 1 read SB1, which the key-block-1 MFMAs of
    S(e+1) overwrite from slot 24, and pair j's pack overwrites the score register of pair
    j // 2, so the pairs run in order); the fp16 row sums in pair order (slots 24..31).  Then
    the row-sum test: a lane-partial row sum of 128 or more (or inf / NaN) sends the wave to
    the iteration's refit block (spread_refit), which returns with P(e), its row sums and
    S(e+1) as the compiled epoch has them.
    """
    X, Y = (P[1], P[0]) if u % 2 == 0 else (P[0], P[1])  # X: S(e) key block 0 -> P(e); Y: P(e-1)
    KB, KA = TX + 1, TX  # K read base (krd + kl0) and the XOR-swizzled address of one k-step

    def sr(i: int) -> int:
        return X + i if i < 16 else SB1 + (i - 16)

    def ring(s: int) -> int:
        return RING + 4 * (s % 3)

    def read(s: int) -> list[str]:
        """Operand of MFMA slot s into ring entry s % 3; slots 32 and 33 are the next iteration's
        0 and 1 (V(e) from V slot (u + 1) % 4, issued after MFMAs 30 and 31 free their entries)."""
        return vread(s, u) if s < 16 else vread(s - 32, (u + 1) % 4) if s >= 32 else kread(s - 16)

    def kread(f: int) -> list[str]:
        s = 16 + f
        blk, kk = f >> 3, f & 7
        # k-step kk reads chunk 2kk + g of the XOR-swizzled row: (krd + kl0) ^ (kk << 5), as krd
        # is a multiple of the 16 KiB tile and the swizzle touches bits 5..7 only
        if kk == 0:
            return [f"ds_read_b128 {v(ring(s), 4)}, {v(KB)} offset:{blk * 8192}"]
        return [f"v_xor_b32 {v(KA)}, {kk << 5}, {v(KB)}",
                f"ds_read_b128 {v(ring(s), 4)}, {v(KA)} offset:{blk * 8192}"]

    def mfma(s: int) -> str:
        if s < 16:
            c = s
            return (f"v_mfma_f32_32x32x16_f16 {v(O + 16 * (c & 3), 16)}, {v(ring(s), 4)}, "
                    f"{v(Y + 4 * (c >> 2), 4)}, {v(O + 16 * (c & 3), 16)}")
        f = s - 16
        dst = Y if f < 8 else SB1
        kk = f & 7
        src_c = "0" if kk == 0 else v(dst, 16)
        return f"v_mfma_f32_32x32x16_f16 {v(dst, 16)}, {v(ring(s), 4)}, {v(Q + 4 * kk, 4)}, {src_c}"

    slots: list[list[str]] = [[] for _ in range(32)]
    # ---- exponential pairs, in place: s -> s * cs - m_run -> exp2 -> fp16 pair in P register j ----
    _spread(exp_stream(X), slots, 1, 23)  # slot 0 holds a K copy (0..23: 0.2-0.6 % slower)
    # ---- fp16 row sums (dot2 with 1.0h) in pair order 0..15 ----
    _spread(row_sums(X), slots, 24, 31)
    # ---- copies: K(e+2) into the K slot kwr (before the iteration's vmcnt), V(e+2) into V slot
    # (u + 3) % 4 (it held V(e-2), last read in the iteration before); the K read base ----
    vw = (3 + (u + 3) % 4) * TILE
    slots[0] = ["s_add_u32 m0, %[ldsw], %[kwr]", "s_nop 0", "global_load_lds_dwordx4 %[ko0], %[kb]",
                "v_add_u32 %[ko0], %[kt2], %[ko0]"] + slots[0]
    slots[2] = ["s_add_u32 m0, %[ldsw], %[kwr]", "s_add_u32 m0, m0, 8192", "s_nop 0",
                "global_load_lds_dwordx4 %[ko1], %[kb]", "v_add_u32 %[ko1], %[kt2], %[ko1]"] + slots[2]
    slots[25] += [f"s_add_u32 m0, %[ldsw], {vw}", "s_nop 0", "global_load_lds_dwordx4 %[vo0], %[vb]",
                  "v_add_u32 %[vo0], %[vt2], %[vo0]"]
    slots[28] += [f"s_add_u32 m0, %[ldsw], {vw + 8192}", "s_nop 0", "global_load_lds_dwordx4 %[vo1], %[vb]",
                  "v_add_u32 %[vo1], %[vt2], %[vo1]"]
    slots[11] += [f"v_add_u32 {v(KB)}, %[krd], %[kl0]"]

    # the reads of slots 0 and 1 were issued by the iteration before (or the scores of epoch 1)
    L = [f"v_mov_b32 {v(LS)}, 0"]
    issued = [0, 0, 1, 1]  # slot of every LDS read in flight, in issue order
    for s in range(32):
        if s + 2 < 32:
            L += read(s + 2)
            issued += [s + 2] * sum(1 for l in read(s + 2) if l.startswith("ds_"))
        last = max(i for i, k in enumerate(issued) if k == s)
        L.append(f"s_waitcnt lgkmcnt({len(issued) - 1 - last})")
        L.append(mfma(s))
        issued = issued[last + 1:]
        if s >= 30:  # next iteration's slots 0 and 1, into the entries MFMAs 30 and 31 read
            L += read(s + 2)
            issued += [s + 2] * 2
        L += slots[s]
    # ---- overflow test on the lane-partial row sums (any lane), then l_run += row sum ----
    L += ["s_nop 2", f"v_cmp_ngt_f32 vcc, {P_CHECK}, {v(LS)}", "s_nop 3",
          f"s_cbranch_vccnz L_refit_{u}_%=", f"L_refitted_{u}_%=:",
          f"v_add_f32 {v(LR)}, {v(LR)}, {v(LS)}"]
    # ---- end: K(e+2) has landed (the V copies may stay in flight), barrier ----
    L += ["s_waitcnt vmcnt(2)", "s_barrier",
          "s_add_u32 %[krd], %[krd], 16384", "s_cmp_eq_u32 %[krd], 49152", "s_cselect_b32 %[krd], 0, %[krd]",
          "s_add_u32 %[kwr], %[kwr], 16384", "s_cmp_eq_u32 %[kwr], 49152", "s_cselect_b32 %[kwr], 0, %[kwr]"]
    return L


def exp_stream(x: int) -> list[str]:
    """The 16 exponential pairs of the scores in x (key block 0, entries 0..15) and SB1 (key
    block 1), in place: s -> s * cs - m_run -> exp2 -> fp16 pair in P register x + j.  Pair t
    is scaled, pair t-1 exponentiated and pair t-2 packed in turn, so two instructions
    separate each exponential from the pack that reads it; P register j is score register j,
    whose pair (j // 2) is done, so the pairs run in order."""
    def sr(i: int) -> int:
        return x + i if i < 16 else SB1 + (i - 16)

    stream = []
    for t in range(18):
        if t < 16:
            stream += [f"v_fma_f32 {v(sr(i))}, {v(sr(i))}, %[cs], -{v(MR)}" for i in (2 * t, 2 * t + 1)]
        if 0 <= t - 1 < 16:
            stream += [f"v_exp_f32 {v(sr(i))}, {v(sr(i))}" for i in (2 * t - 2, 2 * t - 1)]
        if 0 <= t - 2 < 16:
            j = t - 2
            stream += [f"v_cvt_pk_f16_f32 {v(x + j)}, {v(sr(2 * j))}, {v(sr(2 * j + 1))}"]
    return stream


def row_sums(x: int) -> list[str]:
    """The lane-partial fp16 row sum of P (registers x .. x+15) into LS, pairs in order 0..15."""
    return [f"v_dot2c_f32_f16 {v(LS)}, 0x3c003c00, {v(x + j)}" for j in range(16)]


def scores_sequential(kb: str, dst: tuple[int, int]) -> list[str]:
    """S^T of the K tile whose read base (slot + kl0) is in register kb: key block 0 into dst[0],
    key block 1 into dst[1], one fragment read and one MFMA at a time (the rare refit path)."""
    KA = TX
    L = []
    for f in range(16):
        blk, kk = f >> 3, f & 7
        addr = kb
        if kk:
            L.append(f"v_xor_b32 {v(KA)}, {kk << 5}, {kb}")
            addr = v(KA)
        L += [f"ds_read_b128 {v(RING + 4 * (f % 3), 4)}, {addr} offset:{blk * 8192}", "s_waitcnt lgkmcnt(0)"]
        src_c = "0" if kk == 0 else v(dst[blk], 16)
        L.append(f"v_mfma_f32_32x32x16_f16 {v(dst[blk], 16)}, {v(RING + 4 * (f % 3), 4)}, "
                 f"{v(Q + 4 * kk, 4)}, {src_c}")
    return L


def spread_refit(u: int) -> list[str]:
    """The refit block of iteration u, placed after the loop: a lane's row sum of P(e) reached
    128, so the compiled epoch's lazy rescale may fire.  S(e) is recomputed from K(e) (its K
    slot is the one before krd; it is refilled only after the iteration's barrier) into X and
    SB1; the row max over the lane pair gives m_tile, and when any lane has m_tile > m_run + 8
    the compiled epoch's update follows: m_new = max(m_run, m_tile), alpha = exp2(m_run - m_new)
    (1 when m_new = -inf), l_run and O (which holds the tiles before e) scaled by alpha.  P(e)
    and its row sums are recomputed in the main path's order (unchanged values when the rescale
    did not fire); S(e+1) (overwritten) is recomputed from K(e+1) into Y and SB1, and the two V
    fragment reads the next iteration starts with are issued again."""
    X, Y = (P[1], P[0]) if u % 2 == 0 else (P[0], P[1])
    KB = TX + 1
    L = [f"L_refit_{u}_%=:", "s_waitcnt lgkmcnt(0)", "s_nop 7", "s_nop 7", "s_nop 7",
         "s_cmp_eq_u32 %[krd], 0", "s_cselect_b32 %[flag], 49152, %[krd]",
         "s_sub_u32 %[flag], %[flag], 16384",                  # K(e)'s slot
         f"v_add_u32 {v(KB)}, %[flag], %[kl0]"]
    L += scores_sequential(v(KB), (X, SB1))
    L += ["s_nop 7", "s_nop 7", "s_nop 7"]
    # row max of S(e): key block 0 into MX, key block 1 into TMP, then the lane pair
    L += block0_max(X)
    L += [f"v_max3_f32 {v(TMP)}, {v(SB1)}, {v(SB1 + 1)}, {v(SB1 + 2)}"]
    L += [f"v_max3_f32 {v(TMP)}, {v(TMP)}, {v(SB1 + k)}, {v(SB1 + k + 1)}" for k in range(3, 15, 2)]
    L += [f"v_max3_f32 {v(MX)}, {v(MX)}, {v(SB1 + 15)}, {v(TMP)}",
          f"v_mov_b32 {v(TMP)}, {v(MX)}", "s_nop 1", f"v_permlane32_swap_b32 {v(MX)}, {v(TMP)}",
          f"v_max_f32 {v(MX)}, {v(MX)}, {v(TMP)}",
          f"v_mul_f32 {v(MX)}, %[cs], {v(MX)}",                 # m_tile
          f"v_add_f32 {v(TMP)}, 0x41000000, {v(MR)}",            # m_run + 8
          f"v_cmp_gt_f32 vcc, {v(MX)}, {v(TMP)}", "s_nop 3",
          f"s_cbranch_vccz L_kept_{u}_%=",
          f"v_max_f32 {v(TMP)}, {v(MR)}, {v(MX)}",               # m_new
          f"v_sub_f32 {v(ALPHA)}, {v(MR)}, {v(TMP)}",
          f"v_exp_f32 {v(ALPHA)}, {v(ALPHA)}",
          f"v_cmp_eq_f32 vcc, {NEG_INF}, {v(TMP)}",              # m_new = -inf: alpha = 1
          f"v_mov_b32 {v(MR)}, {v(TMP)}",
          f"v_cndmask_b32 {v(ALPHA)}, {v(ALPHA)}, 1.0, vcc",
          f"v_mul_f32 {v(LR)}, {v(LR)}, {v(ALPHA)}"]
    L += [f"v_mul_f32 {v(O + r)}, {v(O + r)}, {v(ALPHA)}" for r in range(64)]
    L += [f"L_kept_{u}_%=:"]
    L += [f"v_mov_b32 {v(LS)}, 0"] + exp_stream(X) + row_sums(X) + ["s_nop 2"]
    L += [f"v_add_u32 {v(KB)}, %[krd], %[kl0]"]              # K(e+1)'s slot
    L += scores_sequential(v(KB), (Y, SB1))
    L += ["s_nop 7", "s_nop 7", "s_nop 7"]
    L += vread(0, (u + 1) % 4) + vread(1, (u + 1) % 4)
    L += [f"s_branch L_refitted_{u}_%="]
    return L


def program_spread() -> list[str]:
    """The dense asm body: S(1) first, then `groups` iterations of 4 epochs, each computing the
    scores of the epoch after it; the rare paths after the loop."""
    L = ["s_mov_b32 %[msave], m0", "s_mov_b32 %[cnt], %[groups]",
         "s_mov_b32 %[krd], %[krd0]", "s_mov_b32 %[kwr], %[kwr0]", "s_nop 1"]
    # ---- S(1) = K(1) . Q^T: key block 0 into P region B, key block 1 into SB1 ----
    KB, KA = TX + 1, TX
    # V(2) into V slot 2 (the loop copies V two epochs ahead)
    L += [f"s_add_u32 m0, %[ldsw], {5 * TILE}", "s_nop 0", "global_load_lds_dwordx4 %[vo0], %[vb]",
          f"s_add_u32 m0, %[ldsw], {5 * TILE + 8192}", "s_nop 0", "global_load_lds_dwordx4 %[vo1], %[vb]",
          "v_add_u32 %[vo0], %[vt2], %[vo0]", "v_add_u32 %[vo1], %[vt2], %[vo1]"]
    L += [f"v_add_u32 {v(KB)}, %[krd], %[kl0]"]

    def kread(f: int) -> list[str]:
        blk, kk = f >> 3, f & 7
        if kk == 0:
            return [f"ds_read_b128 {v(RING + 4 * (f % 3), 4)}, {v(KB)} offset:{blk * 8192}"]
        return [f"v_xor_b32 {v(KA)}, {kk << 5}, {v(KB)}",
                f"ds_read_b128 {v(RING + 4 * (f % 3), 4)}, {v(KA)} offset:{blk * 8192}"]

    L += kread(0) + kread(1)
    for f in range(16):
        if f + 2 < 16:
            L += kread(f + 2)
        L.append(f"s_waitcnt lgkmcnt({min(2, 15 - f)})")
        dst = P[1] if f < 8 else SB1
        src_c = "0" if f & 7 == 0 else v(dst, 16)
        L.append(f"v_mfma_f32_32x32x16_f16 {v(dst, 16)}, {v(RING + 4 * (f % 3), 4)}, "
                 f"{v(Q + 4 * (f & 7), 4)}, {src_c}")
    # K(2) and V(1), copied by the epoch before the loop, land for every wave (V(2) may stay in
    # flight); K(2) is next; the first two V(0) fragments of iteration 1
    L += ["s_waitcnt vmcnt(2)", "s_barrier",
          "s_add_u32 %[krd], %[krd], 16384", "s_cmp_eq_u32 %[krd], 49152", "s_cselect_b32 %[krd], 0, %[krd]",
          "s_nop 7", "s_nop 7", "s_nop 7"]
    L += vread(0, 0) + vread(1, 0)
    L += ["L_epochs_%=:"]
    for u in range(4):
        L += spread_iteration(u)
    L += ["s_sub_u32 %[cnt], %[cnt], 1", "s_cmp_lg_u32 %[cnt], 0", "s_cbranch_scc1 L_epochs_%=",
          "s_branch L_done_%="]
    for u in range(4):
        L += spread_refit(u)
    # the compiled code after the statement reads O and reuses the score registers: MFMA
    # result latency first
    # (and the last iteration's two V reads for an iteration that does not come have landed)
    L += ["L_done_%=:", "s_waitcnt lgkmcnt(0)", "s_mov_b32 m0, %[msave]", "s_nop 7", "s_nop 7", "s_nop 7"]
    return L


def program(kmask: bool = False) -> list[str]:
    """The asm body of the loop the kernel runs: the spread dense loop, or the key-masked one."""
    return one_phase_program(True) if kmask else program_spread()


def one_phase_program(kmask: bool = False) -> list[str]:
    """The one-phase asm body: M0 saved, `groups` iterations of 4 epochs, M0 restored."""
    L = ["s_mov_b32 %[msave], m0", "s_mov_b32 %[cnt], %[groups]",
         "s_mov_b32 %[krd], %[krd0]", "s_mov_b32 %[kwr], %[kwr0]", "s_nop 1"]
    L += ["L_epochs_%=:"]
    for u in range(4):
        L += epoch(u, kmask)
    L += ["s_sub_u32 %[cnt], %[cnt], 1", "s_cmp_lg_u32 %[cnt], 0", "s_cbranch_scc1 L_epochs_%="]
    # the compiled code after the statement reads O: MFMA result latency first
    L += ["s_mov_b32 m0, %[msave]", "s_nop 7", "s_nop 7", "s_nop 7"]
    return L


INCS = {False: "tk_attn_epochs.inc", True: "tk_attn_epochs_kmask.inc"}


def render(kmask: bool = False) -> str:
    head = "// Generated by gen_attn_epochs.py%s; do not edit.\n" % (" (key-masked)" if kmask else "")
    body = "\n".join(f'"{l}\\n"' if l.endswith(":") else f'"{l}\\n\\t"' for l in program(kmask))
    return head + body + "\n"


def clobber_list() -> str:
    return ", ".join(f'"v{r}"' for r in CLOBBERED)


def write(directory: pathlib.Path | None = None) -> list[pathlib.Path]:
    paths = []
    for kmask, name in INCS.items():
        path = (directory or pathlib.Path(__file__).resolve().parent) / name
        text = render(kmask)
        if not path.exists() or path.read_text() != text:
            path.write_text(text)
        paths.append(path)
    return paths


if __name__ == "__main__":
    for out, kmask in zip(write(pathlib.Path(sys.argv[1]) if len(sys.argv) > 1 else None), INCS):
        prog = program(kmask)
        print(out, len(prog), "lines", sum(1 for l in prog if l.startswith("v_mfma")), "MFMAs")
