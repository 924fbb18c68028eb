"""The generated steady-state loops of the causal attention: head_dim 128
(transformer-kernel_amd/csrc/gen_attn_epochs.py -> tk_attn_epochs.inc) and
head_dim 64 (gen_attn_steps64.py -> tk_attn_steps64.inc).

CPU checks of the asm text: it is the generator's output, the kernel's clobber list
names exactly the registers it uses beyond its operands, it never writes the
input-only Q fragments, and along every path through the loop (rescale taken or
skipped, back edge included) the hazards the hardware does not interlock get at
least the wait states the compiler gives them for gfx950.  The wait-state
checker is itself checked on planted mistakes.  Bit-identity with the compiled
epochs is a GPU test (tests/test_gpu_kernels.py).
"""

from __future__ import annotations

import importlib.util
import pathlib
import re

import pytest

CSRC = pathlib.Path(__file__).resolve().parents[1] / "transformer-kernel_amd" / "csrc"


def _gen(name):
    spec = importlib.util.spec_from_file_location(name, CSRC / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


gen = _gen("gen_attn_epochs")
gen64 = _gen("gen_attn_steps64")
class _G64:
    """A head_dim-64 loop variant through the common generator interface."""
    CLOBBERED, PINNED = gen64.CLOBBERED, gen64.PINNED

    def __init__(self, nw, kmask):
        self.nw, self.kmask = nw, kmask

    def program(self):
        return gen64.program(self.nw, self.kmask)

    def render(self):
        return gen64.render(self.nw, self.kmask)


class _KMask:
    """The key-masked head_dim-128 loop through the common generator interface."""
    CLOBBERED, PINNED = gen.CLOBBERED, gen.PINNED

    @staticmethod
    def program():
        return gen.program(True)

    @staticmethod
    def render():
        return gen.render(True)


# (generator, its .inc, the first Q register, Q registers)
LOOPS = {"hd128": (gen, gen.INCS[False], gen.Q, 32), "hd128kmask": (_KMask, gen.INCS[True], gen.Q, 32)}
LOOPS.update({f"hd64{'w8' if nw == 8 else ''}{'kmask' if km else ''}": (_G64(nw, km), inc, gen64.Q, 16)
              for (nw, km), inc in gen64.INCS.items()})


@pytest.mark.parametrize("loop", LOOPS)
def test_committed_inc_is_the_generator_output(loop):
    g, inc, _, _ = LOOPS[loop]
    assert (CSRC / inc).read_text() == g.render()


@pytest.mark.parametrize("loop", LOOPS)
def test_kernel_clobber_list_matches_the_generator(loop):
    g, inc, _, _ = LOOPS[loop]
    src = (CSRC / "tk_attention.hip").read_text()
    i = src.index(f'#include "{inc}"')
    stmt = src[i:src.index(");", i)]
    if "OPERANDS" in stmt:  # the operand list is a macro defined just before the statement
        d = src.rindex("#define TK_", 0, i)
        stmt = src[d:i]
    elif "_CLOBS" in stmt:  # outputs, inputs and clobbers are macros defined before the statements
        name = re.search(r"(TK_\w+_CLOBS)", stmt).group(1)
        d = src.rindex(f"#define {name}", 0, i)
        stmt = src[d:src.index("if constexpr", d)] + stmt
    clobbers = [int(r) for r in re.findall(r'"v(\d+)"', stmt)]
    assert sorted(clobbers) == g.CLOBBERED and len(set(clobbers)) == len(clobbers)
    for extra in ('"vcc"', '"scc"', '"memory"'):
        assert extra in stmt


# --------------------------------------------------------------------------- #
# instruction model
# --------------------------------------------------------------------------- #


def _regs(tok: str) -> list[str]:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return [f"v{r}" for r in range(int(m.group(1)), int(m.group(2)) + 1)]
    m = re.fullmatch(r"-?v(\d+)", tok)
    if m:
        return [f"v{m.group(1)}"]
    if tok in ("m0", "vcc"):
        return [tok]
    return []


class Ins:
    def __init__(self, text: str):
        self.text = text
        parts = text.split(None, 1)
        self.op = parts[0]
        ops = [t.strip() for t in parts[1].split(",")] if len(parts) > 1 else []
        ops = [t.split()[0] for t in ops if t]  # drop "offset:..." modifiers
        self.reads: set[str] = set()
        self.writes: set[str] = set()
        self.src_ab: set[str] = set()
        op = self.op
        if op.startswith("s_nop"):
            self.waits = int(ops[0]) + 1
        else:
            self.waits = 1
        if op.startswith("v_mfma"):
            self.writes = set(_regs(ops[0]))
            self.src_ab = set(_regs(ops[1])) | set(_regs(ops[2]))
            self.reads = self.src_ab | set(_regs(ops[3]))
        elif op.startswith("v_cmp"):
            self.writes = {"vcc"}
            self.reads = {r for t in ops[1:] for r in _regs(t)}
        elif op.startswith("v_permlane32_swap"):
            self.writes = self.reads = {r for t in ops for r in _regs(t)}
        elif op.startswith("v_") or op.startswith("ds_read"):
            self.writes = set(_regs(ops[0]))
            self.reads = {r for t in ops[1:] for r in _regs(t)}
            if op.startswith("v_dot2c"):
                self.reads |= self.writes
        elif op.startswith("global_load_lds"):
            self.reads = {"m0"}
        elif op.startswith("s_") and ops and ops[0] == "m0":
            self.writes = {"m0"}
        elif op in ("s_cbranch_vccz", "s_cbranch_vccnz"):
            self.reads = {"vcc"}
        self.target = ops[0] if op.startswith("s_cbranch") or op == "s_branch" else None


def _cfg(lines: list[str]):
    """Instructions and the predecessors of each (forward branches, the loop's back edge)."""
    ins, label_at = [], {}
    for line in lines:
        if line.endswith(":"):
            label_at[line[:-1]] = len(ins)
        else:
            ins.append(Ins(line))
    preds = [set() for _ in ins]
    for i, x in enumerate(ins):
        if i + 1 < len(ins) and x.op != "s_branch":
            preds[i + 1].add(i)
        if x.target is not None:
            preds[label_at[x.target]].add(i)
    return ins, preds


def _rule(prod: Ins, cons: Ins, reg: str) -> int:
    """Wait states needed between a producer writing `reg` and a consumer touching it."""
    p, c = prod.op, cons.op
    touches = reg in cons.reads or reg in cons.writes
    if p.startswith("v_mfma"):
        if c.startswith("v_mfma"):
            return 18 if reg in cons.src_ab else 0  # accumulate chains forward
        return 18 if touches else 0
    if p.startswith("v_dot2c"):
        return 3 if touches and c.startswith("v_") and not c.startswith("v_dot2c") else 0
    if p.startswith("v_exp"):
        return 1 if reg in cons.reads and c.startswith("v_") and not c.startswith("v_exp") else 0
    if reg == "m0":
        return 1 if c.startswith("global_load_lds") else 0
    if reg == "vcc":
        return 4 if c in ("s_cbranch_vccz", "s_cbranch_vccnz") else 0
    if c.startswith("v_permlane32_swap") and p.startswith("v_"):
        return 2 if reg in cons.reads else 0
    return 0


def hazard_violations(lines: list[str], horizon: int = 32) -> list[str]:
    ins, preds = _cfg(lines)
    bad = []
    for ci, cons in enumerate(ins):
        want = cons.reads | cons.writes
        if not want:
            continue
        # backward walk over every path: (instruction, wait states so far, registers not yet shadowed)
        stack = [(p, 0, frozenset(want)) for p in preds[ci]]
        seen = set()
        while stack:
            pi, ws, regs = stack.pop()
            if (pi, ws, regs) in seen or ws > horizon or not regs:
                continue
            seen.add((pi, ws, regs))
            prod = ins[pi]
            hit = regs & prod.writes
            for reg in hit:
                need = _rule(prod, cons, reg)
                if ws < need:
                    bad.append(f"{prod.text!r} -> {cons.text!r} ({reg}): {ws} < {need}")
            rest = regs - hit
            for q in preds[pi]:
                stack.append((q, ws + prod.waits, rest))
    return bad


def _asm_lines(program: list[str]) -> list[str]:
    return [l.replace("%=", "0") for l in program]


@pytest.mark.parametrize("loop", LOOPS)
def test_generated_loop_meets_the_wait_states(loop):
    bad = hazard_violations(_asm_lines(LOOPS[loop][0].program()))
    assert not bad, "\n".join(bad[:10])


@pytest.mark.parametrize("planted", ["dot2c", "exp", "mfma", "m0", "permlane"])
def test_wait_state_checker_finds_planted_mistakes(planted):
    prog = _asm_lines(gen.program())
    if planted == "dot2c":  # the row-sum test right after the last row-sum dot
        i = next(i for i, l in enumerate(prog) if l.startswith("v_cmp_ngt_f32"))
        assert prog[i - 1] == "s_nop 2"
        del prog[i - 1]
    elif planted == "exp":  # a P conversion right after the exponential it reads
        i = next(i for i, l in enumerate(prog) if l.startswith("v_cvt_pk_f16_f32"))
        src = prog[i].split(", ")[-1]
        j = max(k for k in range(i) if prog[k] == f"v_exp_f32 {src}, {src}")
        prog.insert(j + 1, prog[i])
    elif planted == "mfma":  # a score read right after the MFMA that writes it
        sb = f"v[{gen.SB1}:{gen.SB1 + 15}]"
        i = next(i for i, l in enumerate(prog) if l.startswith(f"v_mfma_f32_32x32x16_f16 {sb}"))
        prog.insert(i + 1, f"v_max_f32 v{gen.T0}, v{gen.T0}, v{gen.SB1}")
    elif planted == "m0":
        i = next(i for i, l in enumerate(prog) if l.startswith("global_load_lds"))
        assert prog[i - 1] == "s_nop 0"
        del prog[i - 1]
    else:
        i = next(i for i, l in enumerate(prog) if l.startswith("v_permlane32_swap"))
        assert prog[i - 1] == "s_nop 1"
        del prog[i - 1]
    assert hazard_violations(prog), planted


@pytest.mark.parametrize("loop", LOOPS)
def test_loop_registers_stay_in_its_operands_and_clobbers(loop):
    g, _, q0, nq = LOOPS[loop]
    allowed = {f"v{r}" for r in g.PINNED | set(g.CLOBBERED)}
    q_regs = {f"v{r}" for r in range(q0, q0 + nq)}
    ins, _ = _cfg(_asm_lines(g.program()))
    used = set()
    for x in ins:
        used |= {r for r in x.reads | x.writes if re.fullmatch(r"v\d+", r)}
        assert not (x.writes & q_regs), x.text  # Q is an input-only operand
    assert used <= allowed, sorted(used - allowed)
    # every clobber is used
    assert {f"v{r}" for r in g.CLOBBERED} <= used


def _hd128_refits(prog):
    """Split the dense head_dim-128 loop into its main path and its out-of-line refit blocks
    (from an L_refit_ label to the branch back)."""
    main, refits, cur = [], [], None
    for l in prog:
        if l.startswith("L_refit_"):
            cur = [l]
        elif cur is not None:
            cur.append(l)
            if l.startswith("s_branch L_refitted_"):
                refits.append(cur)
                cur = None
        else:
            main.append(l)
    return main, refits


def test_loop_covers_four_epochs_of_32_mfmas():
    # the dense loop computes S(1) and copies V(2) before the loop
    for prog, extra in ((gen.one_phase_program(), 0), (_hd128_refits(gen.program())[0], 1)):
        assert sum(1 for l in prog if l.startswith("v_mfma")) == 4 * 32 + 16 * extra
        assert sum(1 for l in prog if l == "s_barrier") == 4 + extra
        assert sum(1 for l in prog if l.startswith("global_load_lds")) == 4 * 4 + 2 * extra


def test_dense_loop_takes_the_row_max_only_in_its_refits():
    """The dense head_dim-128 loop's main path has no row max: after each iteration's row sums
    a lane-partial sum of 128 or more (or NaN) branches to that iteration's refit block, which
    recomputes S(e) (16 MFMAs from the K slot before krd) and its row max, applies the compiled
    epoch's lazy rescale (m_tile > m_run + 8 on any lane: m_run, l_run and the 64 O registers
    updated), recomputes P(e) and its row sums with the main path's own instruction sequence,
    recomputes S(e+1) (16 MFMAs from krd) and re-issues the next iteration's first V reads; it
    touches no memory but LDS."""
    main, refits = _hd128_refits(gen.program())
    assert len(refits) == 4
    assert not any(l.startswith(("v_max", "v_permlane")) for l in main)
    tests = [i for i, l in enumerate(main) if l.startswith("v_cmp_ngt_f32")]
    assert [main[i] for i in tests] == [f"v_cmp_ngt_f32 vcc, 0x43000000, v{gen.LS}"] * 4
    for u, r in enumerate(refits):
        X = gen.P[1] if u % 2 == 0 else gen.P[0]
        it = gen.spread_iteration(u)
        assert r[0] == f"L_refit_{u}_%=:" and f"s_cbranch_vccnz L_refit_{u}_%=" in it
        assert not any(l.startswith(("global_", "buffer_", "scratch_", "s_store", "s_load")) for l in r)
        mf = [l for l in r if l.startswith("v_mfma")]
        assert len(mf) == 32
        dsts = [l.split()[1].rstrip(",") for l in mf]
        sb1 = f"v[{gen.SB1}:{gen.SB1 + 15}]"
        assert dsts[:16] == [f"v[{X}:{X + 15}]"] * 8 + [sb1] * 8
        Y = gen.P[0] if u % 2 == 0 else gen.P[1]
        assert dsts[16:] == [f"v[{Y}:{Y + 15}]"] * 8 + [sb1] * 8
        # rescale test and update as the compiled epoch: m_run + 8, any lane, then m_new
        i = r.index(f"v_add_f32 v{gen.TMP}, 0x41000000, v{gen.MR}")
        assert r[i + 1:i + 4] == [f"v_cmp_gt_f32 vcc, v{gen.MX}, v{gen.TMP}", "s_nop 3",
                                  f"s_cbranch_vccz L_kept_{u}_%="]
        kept = r.index(f"L_kept_{u}_%=:")
        o_muls = [l for l in r[i:kept] if l.startswith("v_mul_f32 v") and 64 <= int(l.split()[1][1:-1]) < 128]
        assert len(o_muls) == 64
        # P(e) and its row sums: the main path's exponential and row-sum instructions, in order
        p_ops = ("v_fma_f32", "v_exp_f32", "v_cvt_pk_f16_f32", "v_dot2c_f32_f16")
        assert [l for l in r[kept:] if l.startswith(p_ops)] == [l for l in it if l.startswith(p_ops)]
        assert r[-1] == f"s_branch L_refitted_{u}_%="


def _slots(iteration: list[str]) -> list[list[str]]:
    """An iteration cut at its MFMAs: slot s = the MFMA of slot s and what follows it."""
    out = [[]]
    for l in iteration:
        if l.startswith("v_mfma"):
            out.append([])
        out[-1].append(l)
    return out[1:]


@pytest.mark.parametrize("u", range(4))
def test_spread_loop_reads_each_score_before_it_is_replaced(u):
    """The dense loop's iteration u: key-block-1 scores of S(e) (SB1) are all read before the
    first MFMA of S(e+1) key block 1 overwrites them (slot 24); P(e-1) (region Y) is read by
    the 16 P.V MFMAs before S(e+1) key block 0 overwrites it (slot 16); every score register
    is scaled, exponentiated and packed in that order, pairs in order, each P register packed
    after the score in it was consumed; the row sums add P registers 0..15 in order."""
    X, Y = (gen.P[1], gen.P[0]) if u % 2 == 0 else (gen.P[0], gen.P[1])
    sl = _slots(gen.spread_iteration(u))
    assert len(sl) == 32
    sb = {f"v{r}" for r in range(gen.SB1, gen.SB1 + 16)}
    y = {f"v{r}" for r in range(Y, Y + 16)}
    for s, slot in enumerate(sl):
        for x in map(Ins, slot):
            if x.op.startswith("v_mfma"):
                assert (y <= x.writes) == (16 <= s < 24) and (sb <= x.writes) == (s >= 24), (s, x.text)
                if s < 16:
                    assert x.reads & y
            elif x.reads & sb:
                assert s < 24, (s, x.text)
    body = [Ins(l) for l in gen.spread_iteration(u) if not l.startswith(("v_mfma", "s_", "ds_", "global_"))]
    score = lambda i: f"v{X + i}" if i < 16 else f"v{gen.SB1 + i - 16}"
    seq = {score(i): [] for i in range(32)}
    packs = []
    for x in body:
        if x.op in ("v_fma_f32", "v_exp_f32"):
            (r,) = x.writes
            seq[r].append(x.op)
        elif x.op == "v_cvt_pk_f16_f32":
            packs.append(x)
    assert all(ops == ["v_fma_f32", "v_exp_f32"] for ops in seq.values())
    assert [sorted(p.reads) for p in packs] == [sorted({score(2 * j), score(2 * j + 1)}) for j in range(16)]
    assert [next(iter(p.writes)) for p in packs] == [f"v{X + j}" for j in range(16)]
    dots = [x for x in body if x.op == "v_dot2c_f32_f16"]
    assert [sorted(x.reads - {f"v{gen.LS}"}) for x in dots] == [[f"v{X + j}"] for j in range(16)]


def _hd64_refits(prog):
    """Split the dense head_dim-64 loop into its main path and its refit blocks (the
    instructions between the overflow branch and its L_fits label)."""
    main, refits, cur = [], [], None
    for l in prog:
        if l.startswith("s_cbranch_vccz L_fits_"):
            main.append(l)
            cur = []
        elif cur is not None and l.startswith("L_fits_"):
            refits.append(cur)
            main.append(l)
            cur = None
        elif cur is not None:
            cur.append(l)
        else:
            main.append(l)
    return main, refits


def test_hd64_loop_covers_two_steps_of_16_mfmas():
    prog = gen64.program()
    main, refits = _hd64_refits(prog)
    assert sum(1 for l in prog if l.startswith("v_mfma")) == 2 * 16
    assert not any(l.startswith("v_mfma") for r in refits for l in r)
    assert sum(1 for l in prog if l == "s_barrier") == 2
    assert sum(1 for l in prog if l.startswith("global_load_lds")) == 2 * 4
    # 32 exponentials and 16 packs per step, every row-sum term in order
    temps = tuple(f"v_exp_f32 v{r}," for r in (gen64.T0, gen64.T1, gen64.T2, gen64.T3))
    assert sum(1 for l in main if l.startswith(temps)) == 2 * 32
    sums = [l for l in main if l.startswith(f"v_add_f32 v{gen64.LS}, v{gen64.LS}, ")]
    assert len(sums) == 64  # the fp32 exponentials, one add each, in entry order
    exps = [l.split()[1].rstrip(",") for l in main if l.startswith(temps)]
    assert [l.split()[-1] for l in sums] == exps
    # no row max on the main path: the rescale runs only when a P entry overflows fp16
    assert not any(l.startswith(("v_max", "v_permlane")) for l in main)


def test_hd64_refit_recomputes_p_as_the_step_does():
    """When some P(kt) entry overflows fp16 (its row sum is inf or NaN), the dense step
    takes the row max of S(kt), rescales l and O to m_new = max(m_run, m_tile) and computes
    P(kt) and its row sum again: the same scale, exponential, pack and dot operations on
    the same registers, in the same order, as the step's slots."""
    prog = gen64.program()
    main, refits = _hd64_refits(prog)
    assert len(refits) == 2
    p_ops = ("v_fma_f32", "v_exp_f32", "v_cvt_pk_f16_f32", f"v_add_f32 v{gen64.LS}, v{gen64.LS}")
    steps = [[], []]
    k = 0
    for l in main:
        if l.startswith("s_cbranch_vccz L_fits_"):
            k += 1
        elif k < 2 and l.startswith(p_ops):
            steps[k].append(l)
    for par in (0, 1):
        r = refits[par]
        s_cur = gen64.X if par == 0 else gen64.Y
        maxes = [l for l in r if l.startswith(("v_max3_f32", "v_max_f32 v212, v212, v1"))]
        regs = sorted(int(x) for l in maxes for x in re.findall(r"v(\d+)", l)[1:] if int(x) != gen64.MX)
        assert regs == list(range(s_cur, s_cur + 32))
        reset = r.index(f"v_mov_b32 v{gen64.LS}, 0")
        assert [l for l in r[reset:] if l.startswith(p_ops)] == steps[par]
        assert r.index(f"v_mov_b32 v{gen64.MR}, v{gen64.TMP}") < reset
        o_muls = [l for l in r if l.startswith("v_mul_f32 v") and int(l.split()[1][1:-1]) in range(64, 96)]
        assert len(o_muls) == 32
    # the overflow test reads the finished row sum: >= 65504 (the fp16 maximum) or NaN refit
    assert sum(1 for l in main if l == f"v_cmp_ngt_f32 vcc, 0x477fe000, v{gen64.LS}") == 2


def test_hd64_loops_differ_only_in_the_copies():
    four, eight = gen64.program(4), gen64.program(8)
    strip = lambda prog: [l for l in prog if not l.startswith(("global_load_lds", "s_add_u32 m0, m0"))
                          and "%[ko1]" not in l and "%[vo1]" not in l and l != "s_nop 0"]
    assert strip(four) == strip(eight)
    assert sum(1 for l in four if l.startswith("global_load_lds")) == 2 * sum(
        1 for l in eight if l.startswith("global_load_lds"))


def test_key_masked_loop_adds_only_the_mask_work():
    """The key-masked loop is the one-phase dense loop plus, per epoch, the validity-byte load,
    the key bits, 32 score selects and the m = -inf guard."""
    dense, masked = gen.one_phase_program(False), gen.program(True)
    extra = [l for l in masked if l not in dense]
    assert all(l.startswith(("global_load_ubyte", "v_add_u32 %[koff]", "s_waitcnt vmcnt(4)", "v_cmp_",
                             "s_mov_b32 s9", "s_mov_b64 s[94:95]", "s_bfe_i32", "v_cndmask_b32",
                             "v_mov_b32 v196, 0xff800000")) for l in extra), extra[:5]
    # per epoch: 32 score selects and the m = -inf guard's 2 (masked only), and the
    # rescale's alpha = 1 select for m_new = -inf (both loops)
    assert sum(1 for l in dense if l.startswith("v_cndmask_b32")) == 4
    assert sum(1 for l in masked if l.startswith("v_cndmask_b32")) == 4 * (32 + 2 + 1)
    it = iter(masked)  # the dense loop is a subsequence of the masked one, in order
    assert all(any(m == l for m in it) for l in dense)
    src = (CSRC / "tk_attention.hip").read_text()
    i = src.index(f'#include "{gen.INCS[True]}"')
    clobs = src[i:src.index(");", i)]
    assert all(f'"s{r}"' in clobs for r in gen.S_CLOBBERED)


@pytest.mark.parametrize("nw", [4, 8])
def test_hd64_key_masked_loop_adds_only_the_mask_work(nw):
    """The key-masked head_dim-64 loop keeps every instruction of the dense one's main path
    in order; in place of the dense end-of-step overflow test it rescales at the start of
    the step (the lazy test on the row max of the masked scores, O scaled at the step end),
    and it adds the byte load, key bits, the selects and the m = -inf guard."""
    # V fragment reads: the dense loop forms its two V bases once per step, the key-masked
    # loop (whose v160/v163 hold validity bytes) one address per read
    vaddr = lambda prog: [re.sub(r"^(ds_read_b64_tr_b16 v\[\d+:\d+\]), v\d+", r"\1, *", l) for l in prog]
    dense, _ = _hd64_refits(gen64.program(nw, False))
    dense = [l for l in vaddr(dense) if not l.startswith(("v_add_u32 v160, %[vrd]", "v_add_u32 v163, %[vrd]"))]
    masked = vaddr(gen64.program(nw, True))
    check = (f"v_cmp_ngt_f32 vcc, 0x477fe000, v{gen64.LS}", "s_nop 3")
    kept = [l for l in dense if not l.startswith(("s_cbranch_vccz L_fits_", "L_fits_")) and l not in check]
    it = iter(masked)
    assert all(any(m == l for m in it) for l in kept)
    extra = [l for l in masked if l not in kept]
    assert all(l.startswith(("global_load_ubyte", "v_add_u32 %[koff]", "v_add_u32 v21", "s_waitcnt vmcnt", "v_cmp_",
                             "s_mov_b32 s9",
                             "s_mov_b64 s[94:95]", "s_mov_b64 s[92:93], %[kbits]", "s_bfe_i32", "v_cndmask_b32", "v_mov_b32 v", "v_max",
                             "v_permlane32_swap", "v_mul_f32", "v_add_f32 v213", "v_sub_f32", "v_exp_f32 v216",
                             "s_nop", "s_cbranch_vccz L_norescale", "L_norescale", "s_mov_b32 %[flag]",
                             "s_cmp_eq_u32 %[flag]", "s_cbranch_scc1 L_noscale", "L_noscale")) for l in extra), extra
    maxes = [l for l in masked if l.startswith("v_max3_f32 v212")]
    assert len(maxes) == 2 * 15
    assert sum(1 for l in masked if l.startswith("s_bfe_i32")) == 2 * 2 * 32
    src = (CSRC / "tk_attention.hip").read_text()
    i = src.index(f'#include "{gen64.INCS[(nw, True)]}"')
    clobs = src[i:src.index(");", i)]
    assert all(f'"s{r}"' in clobs for r in gen64.KMASK_SGPRS)
