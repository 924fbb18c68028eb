"""Emit tk_attn_steps64{,_w8}.inc: the hand-ordered steady-state steps of the head_dim-64 causal
attention (flash_dma_body in tk_attention.hip; 4 waves and 128 query rows per workgroup up to
32768 keys, 8 waves and 256 rows beyond -- the two differ only in the copies per wave).

    python gen_attn_steps64.py [directory]    # default: beside this file

The build runs this before compiling tk_attention.hip.

What a step computes
--------------------
Step kt of the DMA body (key tile kt = keys 64kt .. 64kt+63), for every wave:

  16 slots  slot m < 8: S^T(kt+1) MFMA m (key block m / 4, k-step m % 4);
            slot m >= 8: O^T += V^T(kt-1) . P^T(kt-1), MFMA m - 8 (head-dim block (m-8) % 2,
            P block (m-8) / 2); exponential pair m of S(kt) (entries 2m, 2m+1) between the
            MFMAs -> P(kt) = exp2(cs*S(kt) - m_run) in fp16, row sum of the fp32 exponentials
  copies    K tile kt+2 after slot 0, V tile kt+1 after slot 2 (LDS DMA)
  fit       the reference m_run moves only when the row sum reaches 65504, the fp16 maximum
            (so before any P(kt) entry could overflow fp16; a NaN also lands here): then
            m_tile = cs * (row max of
            S(kt) over the lane pair), m_new = max(m_run, m_tile), alpha = exp2(m_run - m_new),
            l_run *= alpha, O *= alpha (O holds tiles < kt), and P(kt) and its row sum again
  end       l_run += row sum; wait for this step's copies; barrier

No row max is taken on the common path (the max chain and the rescale test were ~20 of a step's
~130 VALU instructions; the step is VALU-bound).  Exponentials up to 2^16 keep fp16's relative
precision, and O, l accumulate in fp32, so a reference up to 16 below the row max costs nothing.
The key-masked loops keep the lazy test at the step start (rescale when any lane's m_tile, from
the masked scores, exceeds m_run + 8; O *= alpha at the step end), since m_run may still be -inf.

Each lane performs the compiled step's operations on the same operands in the same order (the
MFMA accumulation chains, the exponentials, the fp16 packing and the row-sum order; the row max
is exact in any order), so the results are bit-identical to it.  The loop runs steps
[1, 1 + 2*groups), which the host side chooses so that no key tile in them needs a mask and
every copy is a whole tile.  Without a key mask m_run is finite there (step 0 saw key 0); with
one, every row of the workgroup has seen the same keys with the same validity (no causal mask
applies in these steps), so m_run and m_tile are -inf for all rows of a wave or for none and the
wave-wide rescale test never fires for a row whose m_new would be -inf.  The rescale still maps
m_new = -inf to alpha = 1 (one compare and one select on that rare path), so l and O cannot turn
into NaN if the loop's gate ever admits rows with different key histories.  Two steps per
iteration: the score and P registers swap roles between them (the compiled loop's s_a/s_b,
pf_a/pf_b), the K slot (2 slots) follows the parity and the V slots (3) rotate through SGPR
trackers.

Register map (VGPRs; the asm statement pins or clobbers every one of them)
--------------------------------------------------------------------------
  v[64:95]    O^T accumulators, 2 x 16                     (in/out)
  v[96:111]   Q fragments, 4 x 4                            (in)
  v[112:143]  scores X: S(kt) at entry and exit             (in/out)
  v[144:159]  P tile W: P(kt-1) at entry and exit           (in/out)
  v160        dense: V read base of head-dim block 0;       (in/out; dead after the loop)
              key-masked: validity bytes of the next tile
  v161, v162  m_run, l_run                                  (in/out)
  v163        dense: V read base of head-dim block 1;       (clobbered)
              key-masked: validity bytes (other parity)
  v[164:195]  scores Y                                      (clobbered)
  v[196:211]  P tile Z                                      (clobbered)
  v212..v217  temporaries                                   (clobbered)
  v[218:229]  operand ring, 3 x 4 (K or V fragments)         (clobbered)

Wait states: as in gen_attn_epochs.py (M0 -> LDS DMA 1, MFMA -> VALU 24 or an MFMA-free
stretch of at least 18 instructions, VALU -> v_permlane32_swap 2, VCC -> s_cbranch_vccz 4,
v_exp -> VALU 1).
"""
from __future__ import annotations

import pathlib
import sys

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
from gen_attn_epochs import NEG_INF, S_CLOBBERED, S_KB, S_NOKEY, key_mask  # noqa: E402

O = 64
Q = 96
X, W, MXX = 112, 144, 160
MR, LR = 161, 162
MXY, Y, Z = 163, 164, 196
T0, T1, T2, T3 = 212, 213, 214, 215   # exponential pipeline, two pairs
MX, TMP = T0, T1                      # the max phase ends before the pipeline starts
ALPHA, LS = 216, 217
RING = 218                            # 64-bit aligned tuples
FP16_MAX = "0x477fe000"                # 65504.0
VA = (MXX, MXY)                       # dense loops: this step's V read bases (head-dim blocks 0, 1)
TILE = 8192                           # bytes per K or V tile (64 rows x 128 bytes)
KSLOTS, VSLOTS = 2, 3

PINNED = set(range(64, 160)) | {MXX, MR, LR}
CLOBBERED = sorted({MXY} | set(range(164, 230)))


def v(a: int, n: int = 1) -> str:
    return f"v{a}" if n == 1 else f"v[{a}:{a + n - 1}]"


def row_max(s: int) -> list[str]:
    """Row max of the 32 scores s[0:32] of this lane, then over the lane pair, times cs: MX =
    m_tile (TMP clobbered)."""
    L = [f"v_max3_f32 {v(MX)}, {v(s)}, {v(s + 1)}, {v(s + 2)}"]
    for k in range(3, 31, 2):
        L.append(f"v_max3_f32 {v(MX)}, {v(MX)}, {v(s + k)}, {v(s + k + 1)}")
    return L + [f"v_max_f32 {v(MX)}, {v(MX)}, {v(s + 31)}", f"v_mov_b32 {v(TMP)}, {v(MX)}", "s_nop 1",
                f"v_permlane32_swap_b32 {v(MX)}, {v(TMP)}",
                f"v_max_f32 {v(MX)}, {v(MX)}, {v(TMP)}",
                f"v_mul_f32 {v(MX)}, {v(MX)}, %[cs]"]


def rescale(tag: str, flag: str | None = None) -> list[str]:
    """m_new = max(m_run, m_tile), alpha = exp2(m_run - m_new) (1 for m_new = -inf), l_run *=
    alpha.  With flag (the lazy test of the key-masked steps): only when some lane's m_tile
    exceeds m_run + 8, and the flag asks for O *= alpha at the end of the step."""
    L = []
    if flag:
        L += [f"v_add_f32 {v(TMP)}, 0x41000000, {v(MR)}",             # m_run + 8
              f"v_cmp_gt_f32 vcc, {v(MX)}, {v(TMP)}", "s_nop 3",
              f"s_cbranch_vccz L_norescale_{tag}_%="]
    L += [f"v_max_f32 {v(TMP)}, {v(MR)}, {v(MX)}",                     # m_new
          f"v_sub_f32 {v(ALPHA)}, {v(MR)}, {v(TMP)}",
          f"v_exp_f32 {v(ALPHA)}, {v(ALPHA)}",
          f"v_cmp_eq_f32 vcc, {NEG_INF}, {v(TMP)}",                    # m_new = -inf: alpha = 1
          f"v_mov_b32 {v(MR)}, {v(TMP)}",
          f"v_cndmask_b32 {v(ALPHA)}, {v(ALPHA)}, 1.0, vcc",
          f"v_mul_f32 {v(LR)}, {v(LR)}, {v(ALPHA)}"]
    if flag:
        L += [flag, f"L_norescale_{tag}_%=:"]
    return L


def o_scale() -> list[str]:
    return [f"v_mul_f32 {v(O + r)}, {v(O + r)}, {v(ALPHA)}" for r in range(32)]


def step(par: int, nw: int = 4, kmask: bool = False) -> list[str]:
    """One step of an nw-wave workgroup (4: two 1 KB copies per tile and wave, 8: one);
    par 0: scores X current, Y next, P W previous, Z new; par 1 swaps them.
    Step kt has par = (kt + 1) % 2 (the loop starts at kt = 1).

    kmask (key-validity mask): like the compiled key-masked step, the row max of S(kt) is taken
    over its scores after the invalid keys' scores are set to -inf (s92/s93 hold tile kt's key
    bits), so the next tile's running max is not kept, and its register takes the next tile's
    validity bytes (loaded at the start of the step, turned into key bits after its copy wait);
    rows with no valid key yet exponentiate against 0 and keep m = -inf."""
    s_cur, s_nxt = (X, Y) if par == 0 else (Y, X)
    p_prev, p_cur = (W, Z) if par == 0 else (Z, W)
    kb_nxt = MXY if par == 0 else MXX      # key-masked: the next tile's validity bytes
    k_rd = par * TILE                     # K(kt+1) is read from slot (kt + 1) % 2 = par
    k_wr = (1 - par) * TILE               # K(kt+2) is written into slot kt % 2

    L = ["s_mov_b32 %[flag], 0"] if kmask else [f"v_add_u32 {v(VA[d])}, %[vrd], %[vl{d}]" for d in (0, 1)]
    L += [f"v_mov_b32 {v(LS)}, 0"]
    if kmask:
        L += [f"global_load_ubyte {v(kb_nxt)}, %[koff], %[kvb]", "v_add_u32 %[koff], 64, %[koff]"]
        # ---- row max of S(kt) after the mask, over the lane pair; lazy rescale ----
        L += key_mask(lambda i: s_cur + i, ALPHA)
        L += row_max(s_cur) + rescale(f"{par}", "s_mov_b32 %[flag], 1")
    if kmask:  # rows with no valid key so far: exponentials against 0, m_run restored after
        L += [f"v_cmp_eq_f32 vcc, {NEG_INF}, {v(MR)}", f"s_mov_b64 s[{S_NOKEY}:{S_NOKEY + 1}], vcc",
              f"v_cndmask_b32 {v(MR)}, {v(MR)}, 0, vcc"]
    # ---- fragment reads: slot m's fragment into ring entry m % 3; read addresses go
    # through the exponential pair that is idle where the read is issued (ka) ----
    def reads(m: int, ka: int = -1) -> list[str]:
        r = RING + 4 * (m % 3)
        if m < 8:
            kb2, kk = m // 4, m % 4
            off = k_rd + kb2 * 4096
            return [f"ds_read_b128 {v(r, 4)}, %[kl{kk}] offset:{off}"]  # kl{kk} = kl0 ^ (kk << 5)
        c = m - 8
        t, d = c // 2, c % 2
        if not kmask:  # this step's V slot base, formed at the step start
            return [f"ds_read_b64_tr_b16 {v(r, 2)}, {v(VA[d])} offset:{t * 2048}",
                    f"ds_read_b64_tr_b16 {v(r + 2, 2)}, {v(VA[d])} offset:{t * 2048 + 1024}"]
        return [f"v_add_u32 {v(ka)}, %[vrd], %[vl{d}]",
                f"ds_read_b64_tr_b16 {v(r, 2)}, {v(ka)} offset:{t * 2048}",
                f"ds_read_b64_tr_b16 {v(r + 2, 2)}, {v(ka)} offset:{t * 2048 + 1024}"]

    def n_ds(m: int) -> int:
        return 1 if m < 8 else 2

    # ---- exponential pipeline over the slots (pair j: entries 2j, 2j+1 of S(kt)) ----
    tp = ((T0, T1), (T2, T3))

    def sr(i: int) -> int:
        return s_cur + i

    def scale(j: int) -> list[str]:
        a, b = tp[j % 2]
        return [f"v_fma_f32 {v(a)}, {v(sr(2 * j))}, %[cs], -{v(MR)}",
                f"v_fma_f32 {v(b)}, {v(sr(2 * j + 1))}, %[cs], -{v(MR)}"]

    def expo(j: int) -> list[str]:
        a, b = tp[j % 2]
        return [f"v_exp_f32 {v(a)}, {v(a)}", f"v_exp_f32 {v(b)}, {v(b)}"]

    def pack(j: int) -> list[str]:
        a, b = tp[j % 2]
        return [f"v_cvt_pk_f16_f32 {v(p_cur + j)}, {v(a)}, {v(b)}",   # P(kt) pair j in fp16
                f"v_add_f32 {v(LS)}, {v(LS)}, {v(a)}",                   # row sum of the fp32
                f"v_add_f32 {v(LS)}, {v(LS)}, {v(b)}"]                   # exponentials, in order

    # ---- copies ----
    # copy i of wave w fills LDS bytes (w + i*nw) * 1024 of the slot
    cpw = (TILE // 1024) // nw
    kcopy = ["s_add_u32 m0, %[ldsw], " + str(k_wr), "s_nop 0", "global_load_lds_dwordx4 %[ko0], %[kb]"]
    vcopy = ["s_add_u32 m0, %[ldsw], %[vwr]", f"s_add_u32 m0, m0, {KSLOTS * TILE}", "s_nop 0",
             "global_load_lds_dwordx4 %[vo0], %[vb]"]
    for i in range(1, cpw):
        kcopy += [f"s_add_u32 m0, m0, {nw * 1024}", "s_nop 0", f"global_load_lds_dwordx4 %[ko{i}], %[kb]"]
        vcopy += [f"s_add_u32 m0, m0, {nw * 1024}", "s_nop 0", f"global_load_lds_dwordx4 %[vo{i}], %[vb]"]
    kcopy += [f"v_add_u32 %[ko{i}], %[kt2], %[ko{i}]" for i in range(cpw)]
    vcopy += [f"v_add_u32 %[vo{i}], %[vt2], %[vo{i}]" for i in range(cpw)]

    # ---- the 16 slots ----
    RA = 2
    for m in range(RA):
        L += reads(m, tp[1][0])    # pair 1 is free until scale(1) in slot 0
    L += scale(0)
    for m in range(16):
        if m + RA < 16:
            L += reads(m + RA, tp[(m + 1) % 2][0])  # pack(m-1) has read it, scale(m+1) comes later
        pending = sum(n_ds(k) for k in range(m + 1, min(16, m + RA + 1)))
        L.append(f"s_waitcnt lgkmcnt({pending})")
        r = RING + 4 * (m % 3)
        if m < 8:
            kb2, kk = m // 4, m % 4
            src_c = "0" if kk == 0 else v(s_nxt + 16 * kb2, 16)
            L.append(f"v_mfma_f32_32x32x16_f16 {v(s_nxt + 16 * kb2, 16)}, {v(r, 4)}, {v(Q + 4 * kk, 4)}, {src_c}")
        else:
            c = m - 8
            t, d = c // 2, c % 2
            L.append(f"v_mfma_f32_32x32x16_f16 {v(O + 16 * d, 16)}, {v(r, 4)}, {v(p_prev + 4 * t, 4)}, "
                     f"{v(O + 16 * d, 16)}")
        L += expo(m)
        L += scale(m + 1) if m + 1 < 16 else ["s_nop 1"]
        L += pack(m)
        if m == 0:
            L += kcopy
        if m == 2:
            L += vcopy
    L += ["s_nop 2"]
    if not kmask:
        # ---- the row sum reached the fp16 maximum (an entry of P(kt) may have overflowed; or
        # NaN): the row max of S(kt), the rescale of l and O, P(kt) and its row sum again ----
        L += [f"v_cmp_ngt_f32 vcc, {FP16_MAX}, {v(LS)}", "s_nop 3", f"s_cbranch_vccz L_fits_{par}_%="]
        L += row_max(s_cur) + rescale(f"{par}") + ["s_nop 7", "s_nop 7", "s_nop 7"] + o_scale()
        L += [f"v_mov_b32 {v(LS)}, 0"] + scale(0)
        for j in range(16):
            L += expo(j) + (scale(j + 1) if j + 1 < 16 else ["s_nop 1"]) + pack(j)
        L += ["s_nop 2", f"L_fits_{par}_%=:"]
    L += [f"v_add_f32 {v(LR)}, {v(LR)}, {v(LS)}"]
    if kmask:  # ---- O rescale ----
        L += ["s_cmp_eq_u32 %[flag], 0", f"s_cbranch_scc1 L_noscale_{par}_%=", "s_nop 7", "s_nop 7", "s_nop 7"]
        L += o_scale() + [f"L_noscale_{par}_%=:"]
    if kmask:
        L += [f"v_mov_b32 {v(ALPHA)}, {NEG_INF}",
              f"v_cndmask_b32 {v(MR)}, {v(MR)}, {v(ALPHA)}, s[{S_NOKEY}:{S_NOKEY + 1}]"]
    # ---- end: this step's copies have landed; barrier; next V slots ----
    L += ["s_waitcnt vmcnt(0) lgkmcnt(0)"]
    if kmask:  # the next tile's key bits
        L += [f"v_cmp_ne_u32 vcc, 0, {v(kb_nxt)}", f"s_mov_b32 s{S_KB[0]}, vcc_lo",
              f"s_mov_b32 s{S_KB[1]}, vcc_hi"]
    L += ["s_barrier",
          f"s_add_u32 %[vrd], %[vrd], {TILE}", f"s_cmp_eq_u32 %[vrd], {VSLOTS * TILE}",
          "s_cselect_b32 %[vrd], 0, %[vrd]",
          f"s_add_u32 %[vwr], %[vwr], {TILE}", f"s_cmp_eq_u32 %[vwr], {VSLOTS * TILE}",
          "s_cselect_b32 %[vwr], 0, %[vwr]"]
    return L


def program(nw: int = 4, kmask: bool = False) -> list[str]:
    """M0 saved, `groups` iterations of two steps, M0 restored."""
    # the scores and P tile handed in were written by MFMAs and VALU ops of the compiled code
    L = ["s_mov_b32 %[msave], m0", "s_mov_b32 %[cnt], %[groups]", "s_nop 7", "s_nop 7", "s_nop 7"]
    if kmask:  # key bits of tile 1, from the compiled step 0
        L += [f"s_mov_b64 s[{S_KB[0]}:{S_KB[1]}], %[kbits]"]
    L += ["L_steps_%=:"]
    L += step(0, nw, kmask) + step(1, nw, kmask)
    L += ["s_sub_u32 %[cnt], %[cnt], 1", "s_cmp_lg_u32 %[cnt], 0", "s_cbranch_scc1 L_steps_%="]
    # the compiled code after the statement reads O and the scores: MFMA result latency first
    L += ["s_mov_b32 m0, %[msave]", "s_nop 7", "s_nop 7", "s_nop 7"]
    return L


INCS = {(4, False): "tk_attn_steps64.inc", (8, False): "tk_attn_steps64_w8.inc",
        (4, True): "tk_attn_steps64_kmask.inc", (8, True): "tk_attn_steps64_w8_kmask.inc"}
INC = INCS[(4, False)]
KMASK_SGPRS = S_CLOBBERED


def render(nw: int = 4, kmask: bool = False) -> str:
    head = f"// Generated by gen_attn_steps64.py ({nw} waves{', key-masked' if kmask else ''}); do not edit.\n"
    body = "\n".join(f'"{l}\\n"' if l.endswith(":") else f'"{l}\\n\\t"' for l in program(nw, kmask))
    return head + body + "\n"


def write(directory: pathlib.Path | None = None) -> list[pathlib.Path]:
    paths = []
    for (nw, kmask), name in INCS.items():
        path = (directory or pathlib.Path(__file__).resolve().parent) / name
        text = render(nw, kmask)
        if not path.exists() or path.read_text() != text:
            path.write_text(text)
        paths.append(path)
    return paths


if __name__ == "__main__":
    for out, (nw, kmask) in zip(write(pathlib.Path(sys.argv[1]) if len(sys.argv) > 1 else None), INCS):
        prog = program(nw, kmask)
        print(out, len(prog), "lines", sum(1 for l in prog if l.startswith("v_mfma")), "MFMAs")
