"""CPU checks of the wide-tile wgrad kernel's generated assembly (ggemm-asm_amd/csrc/gen_vark_wide.py,
vark_wide.h), before any GPU launch.

The per-tile assembly statement is executed by a small interpreter of its scalar instructions
(SALU arithmetic, compares, branches, m0) that records the vector-memory, LDS and MFMA
instructions as events; the HIP tile loop around it is restated (c0 += nsteps mod 3, the
in/out operands carried). Over many tile sequences (empty tiles, 1-64-token and ragged groups,
long groups) the recorded program must:
  * issue every stage of every tile exactly once, in order, into the slot its reads use, with the
    buffer base and num_records that bound the stage's rows (tokens past the group end read 0);
  * wait (counted vmcnt, in-order completion) for a stage's loads and pass a barrier before any
    wave reads it, and never DMA into a slot before a barrier that follows the last reads of its
    previous stage or of the epilogue staged there, nor stage C in a slot before a barrier that
    follows every read of its stage;
  * issue 24 MFMAs per stage covering the 4 x 6 blocks once (zero accumulator input in a tile's
    first stage), each after the LDS reads of its operands completed (in-order lgkmcnt), and 48 C
    stores per tile whose row/column offsets cover the wave's quadrant;
  * take the same branches and barriers in every wave.
Per-lane address maps (operand reads, LDS-DMA placement, epilogue staging) are checked against
the 32x32x64 operand layout and for LDS bank conflicts.
"""
import importlib.util
import os
import re

import numpy as np
import pytest

from conftest import ROOT

GEN_PATH = os.path.join(ROOT, "ggemm-asm_amd", "csrc", "gen_vark_wide.py")


def _gen():
    spec = importlib.util.spec_from_file_location("gen_vark_wide", GEN_PATH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


GEN = _gen()
M32 = 0xFFFFFFFF


def _program():
    g = GEN.Gen()
    g.tile()
    prog, labels = [], {}
    for line in g.lines:
        if line.endswith(":"):
            labels[line[:-1]] = len(prog)
        else:
            op, _, rest = line.partition(" ")
            args = [a.strip() for a in rest.split(",")] if rest else []
            prog.append((op, args))
    return prog, labels


PROG, LABELS = _program()


def _s32(x):
    x &= M32
    return x - (1 << 32) if x & 0x80000000 else x


class Block:
    """Runs the per-tile statement for one wave with given operand values."""

    def __init__(self, ops, events, scal):
        self.ops = ops          # operand name -> value (SGPR operands) / name (VGPR operands)
        self.ev = events
        self.s = scal           # persistent scalar temporaries (s56..s88), as on the GPU
        self.scc = 0
        self.v = {}             # symbolic VGPR temporaries

    def val(self, a):
        if a.startswith("%"):
            name = GEN.OPERANDS[int(a[1:])][0]
            return self.ops[name]
        if a == "m0":
            return self.s.get("m0", 0)
        if re.fullmatch(r"s\d+", a):
            return self.s[a]
        if a.startswith("0x"):
            return int(a, 16)
        return int(a)

    def setr(self, a, x):
        x &= M32
        if a.startswith("%"):
            name = GEN.OPERANDS[int(a[1:])][0]
            assert GEN.OPERANDS[int(a[1:])][1] == "+s", f"write to input operand {name}"
            self.ops[name] = x
        else:
            assert a == "m0" or re.fullmatch(r"s\d+", a), a
            self.s[a] = x

    def rsrc(self, quad):
        lo, hi = [int(x) for x in re.fullmatch(r"s\[(\d+):(\d+)\]", quad).groups()]
        w = [self.s[f"s{r}"] for r in range(lo, hi + 1)]
        return (w[0] | (w[1] & 0xFFFF) << 32), w[2], w[1] >> 16, w[3]

    def run(self):
        pc = 0
        while pc < len(PROG):
            op, a = PROG[pc]
            pc += 1
            if op in ("s_add_u32", "s_sub_u32", "s_sub_i32", "s_mul_i32", "s_and_b32", "s_lshl_b32",
                      "s_lshr_b32", "s_min_i32", "s_max_i32", "s_min_u32", "s_addc_u32"):
                x, y = self.val(a[1]), self.val(a[2])
                if op == "s_add_u32":
                    r = x + y
                    self.scc = int(r > M32)
                elif op == "s_addc_u32":
                    r = x + y + self.scc
                    self.scc = int(r > M32)
                elif op == "s_sub_u32":
                    r = x - y
                    self.scc = int(r < 0)
                elif op == "s_sub_i32":
                    r = _s32(x) - _s32(y)
                elif op == "s_mul_i32":
                    r = _s32(x) * _s32(y)
                elif op == "s_and_b32":
                    r = x & y
                elif op == "s_lshl_b32":
                    r = x << y
                elif op == "s_lshr_b32":
                    r = x >> y
                elif op == "s_min_i32":
                    r = min(_s32(x), _s32(y))
                elif op == "s_max_i32":
                    r = max(_s32(x), _s32(y))
                else:
                    r = min(x & M32, y & M32)
                self.setr(a[0], r)
            elif op == "s_mov_b32":
                self.setr(a[0], self.val(a[1]))
            elif op in ("s_cmp_eq_u32", "s_cmp_lt_u32", "s_cmp_ge_u32"):
                x, y = self.val(a[0]) & M32, self.val(a[1]) & M32
                self.scc = int(x == y if op == "s_cmp_eq_u32" else x < y if op == "s_cmp_lt_u32" else x >= y)
            elif op == "s_cselect_b32":
                self.setr(a[0], self.val(a[1]) if self.scc else self.val(a[2]))
            elif op == "s_cbranch_scc1":
                if self.scc:
                    pc = LABELS[a[0]]
            elif op == "s_cbranch_scc0":
                if not self.scc:
                    pc = LABELS[a[0]]
            elif op == "s_branch":
                pc = LABELS[a[0]]
            elif op == "s_nop":
                pass
            elif op == "s_barrier":
                self.ev.append(("barrier",))
            elif op == "s_waitcnt":
                m = re.fullmatch(r"(vmcnt|lgkmcnt)\((\d+)\)", a[0])
                self.ev.append((m.group(1), int(m.group(2))))
            elif op == "v_add_u32":
                self.v[a[0]] = (self.val(a[1]), a[2])
            elif op == "buffer_load_dwordx4":
                voff = self.v[a[0]] if a[0] in self.v and not a[0].startswith("%") else (0, a[0])
                self.ev.append(("dma", self.s["m0"], self.rsrc(a[1]), voff, a[-1]))
            elif op == "buffer_store_dwordx4":
                self.ev.append(("store", self.v[a[1]], self.rsrc(a[2]), a[0]))
            elif op == "ds_read_b64_tr_b8":
                reg, mod = a[1].split()
                base = self.v[reg]
                off = int(mod.split(":")[1])
                self.ev.append(("read", base, off, a[0]))
            elif op == "v_mfma_f32_32x32x64_f8f6f4":
                self.ev.append(("mfma", a[0], a[1], a[2], a[3].split()[0]))
            elif op in ("ds_write_b64", "ds_read_b128"):
                self.ev.append((op, a))
            elif op.startswith("v_"):
                pass
            else:
                raise AssertionError(f"interpreter lacks {op}")
        return self


LHS, RHS, OUT = 0x7F0000000000, 0x7E0000000000, 0x7D0000000000


def _run_tiles(tiles, wave, stride_l=2880, stride_r=5760, stride_cm=5760, OUT_M=2880):
    """tiles: list of (g, m0, n0, kb, klen). Returns (events, per-tile event slices, final state)."""
    ev = []
    scal = {f"s{r}": 0 for r in GEN.SGPR_CLOBBER}
    state = dict(c0=0, nis=0, vmt=0, q0=0, q1=0, q2=0, np=0)
    spans = []
    for n, (g, m0, n0, kb, klen) in enumerate(tiles):
        has_next = n + 1 < len(tiles)
        N = tiles[n + 1] if has_next else (0, 0, 0, 0, 0)
        ops = dict(state)
        ops.update(lds_base=0, w1k=1024 * wave,
                   bLT_lo=(LHS + kb * stride_l + m0) & M32, bLT_hi=(LHS + kb * stride_l + m0) >> 32,
                   bRT_lo=(RHS + kb * stride_r + n0) & M32, bRT_hi=(RHS + kb * stride_r + n0) >> 32,
                   klenT=klen, m0T=m0, n0T=n0,
                   bLN_lo=(LHS + N[3] * stride_l + N[1]) & M32, bLN_hi=(LHS + N[3] * stride_l + N[1]) >> 32,
                   bRN_lo=(RHS + N[3] * stride_r + N[2]) & M32, bRN_hi=(RHS + N[3] * stride_r + N[2]) >> 32,
                   klenN=N[4] if has_next else 0, m0N=N[1], n0N=N[2],
                   cT_lo=(OUT + 2 * (m0 * stride_cm + n0)) & M32, cT_hi=(OUT + 2 * (m0 * stride_cm + n0)) >> 32,
                   crecT=((OUT_M - m0) * stride_cm - n0) * 2,
                   stride_l=stride_l, stride_r=stride_r, cm2=2 * stride_cm, alpha=0x3F800000,
                   sw_epi=(128 * (wave & 1) * stride_cm + 192 * (wave >> 1)) * 2)
        start = len(ev)
        Block(ops, ev, scal).run()
        spans.append((start, len(ev)))
        for k in state:
            state[k] = ops[k]
        state["c0"] = (state["c0"] + (klen + 63) // 64) % 3
    return ev, spans, state


def _check(tiles, wave=0, stride_l=2880, stride_r=5760, stride_cm=5760, OUT_M=2880):
    ev, spans, state = _run_tiles(tiles, wave, stride_l, stride_r, stride_cm, OUT_M)
    stages = [(n, s) for n, t in enumerate(tiles) for s in range((t[4] + 63) // 64)]
    slot_of = {st: k % 3 for k, st in enumerate(stages)}
    # ---- DMA: one group of 4 LHS + 6 RHS loads per stage, in stage order
    dmas = [(i, e) for i, e in enumerate(ev) if e[0] == "dma"]
    assert len(dmas) == 10 * len(stages)
    issue_pos = {}
    for k, (n, s) in enumerate(stages):
        g, m0, n0, kb, klen = tiles[n]
        grp = dmas[10 * k:10 * k + 10]
        issue_pos[(n, s)] = (grp[0][0], grp[-1][0])
        rv = min(64, klen - 64 * s)
        for j, (_, e) in enumerate(grp):
            _, m0v, (base, nrec, stride_bits, w3), voff, _ = e
            assert stride_bits == 0 and w3 == GEN.WORD3
            if j < 4:
                assert base == LHS + (kb + 64 * s) * stride_l + m0
                assert nrec == rv * stride_l - m0
                assert m0v == slot_of[(n, s)] * GEN.SLOT + 1024 * wave + 4096 * j
                assert voff == ((0, "%" + str(_opidx("voffL0"))) if j == 0 else (16 * stride_l * j, _op("voffL0")))
            else:
                jj = j - 4
                assert base == RHS + (kb + 64 * s) * stride_r + n0
                assert nrec == rv * stride_r - n0
                assert m0v == slot_of[(n, s)] * GEN.SLOT + GEN.RHS_OFF + 1024 * wave + 4096 * jj
                assert voff == (0, _op(f"voffR{jj}"))
    # ---- reads: groups of 40 in compute order, from the stage's slot
    reads = [(i, e) for i, e in enumerate(ev) if e[0] == "read"]
    assert len(reads) == 40 * len(stages)
    read_span = {}
    for k, st in enumerate(stages):
        grp = reads[40 * k:40 * k + 40]
        read_span[st] = (grp[0][0], grp[-1][0])
        names = []
        for _, (_, (slot_off, name), off, dst) in grp:
            assert slot_off == slot_of[st] * GEN.SLOT, (st, slot_off)
            names.append((name, off))
        want = [(_op(f"amb{i}"), o) for i in range(4) for o in (0, 2048, 8192, 10240)]
        want += [(_op(f"bnb{j}"), o) for j in range(6) for o in (0, 3072, 12288, 15360)]
        assert sorted(names) == sorted(want)
    # ---- completion model: in-order vmcnt, barriers
    issued = []            # event index of each vector-memory op, in order
    done_at = {}           # op index -> event index where it is known complete
    barriers = [i for i, e in enumerate(ev) if e[0] == "barrier"]
    for i, e in enumerate(ev):
        if e[0] in ("dma", "store"):
            issued.append(i)
        elif e[0] == "vmcnt":
            for op_i in issued[:max(len(issued) - e[1], 0)]:
                done_at.setdefault(op_i, i)
    for st in stages:
        first_read = read_span[st][0]
        a, b = issue_pos[st]
        loads = [i for i in issued if a <= i <= b]
        assert all(i in done_at and done_at[i] < first_read for i in loads), f"stage {st} read before its loads"
        last_done = max(done_at[i] for i in loads)
        assert any(last_done < bi < first_read for bi in barriers), f"stage {st}: no barrier after its wait"
    # ---- operand data: every MFMA's A and B registers hold completed reads (in-order lgkmcnt)
    def regs(r):
        m = re.fullmatch(r"v\[(\d+):(\d+)\]", r)
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    pending = []           # (regs written) of issued, not known complete LDS reads
    for e in ev:
        if e[0] == "read":
            pending.append(regs(e[3]))
        elif e[0] in ("ds_write_b64",):
            pending.append(set())
        elif e[0] == "ds_read_b128":
            pending.append(regs(e[1][0]))
        elif e[0] == "lgkmcnt":
            pending = pending[len(pending) - e[1]:] if e[1] < len(pending) else pending
        elif e[0] == "mfma":
            need = regs(e[2]) | regs(e[3])
            assert not any(need & p for p in pending), f"MFMA {e} reads registers of a pending LDS read"
        elif e[0] == "store":
            assert not any(regs(e[3]) & p for p in pending), "store of pending LDS data"
    # ---- slot reuse: a DMA into a slot follows a barrier that follows every read of the previous
    # stage in that slot and every epilogue staging access there
    last_use = {0: -1, 1: -1, 2: -1}
    occupant = {}
    stage_at_dma = {}
    for k, st in enumerate(stages):
        stage_at_dma[issue_pos[st][0]] = st
    epi_slot_events = []
    for n, (a, b) in enumerate(spans):
        if (tiles[n][4] + 63) // 64 > 0:
            last = (n, (tiles[n][4] + 63) // 64 - 1)
            for i in range(a, b):
                if ev[i][0] in ("ds_write_b64", "ds_read_b128"):
                    epi_slot_events.append((i, slot_of[last]))
    uses = []
    for st in stages:
        uses.append((read_span[st][1], slot_of[st]))
    uses += epi_slot_events
    uses.sort()
    for k, st in enumerate(stages):
        pos = issue_pos[st][0]
        slot = slot_of[st]
        prior = [i for i, sl in uses if sl == slot and i < pos]
        if prior:
            assert any(max(prior) < bi < pos for bi in barriers), f"DMA of {st} into slot {slot} races a reader"
        # and no read of this slot's previous stage after the DMA
        later_prev = [i for i, sl in uses if sl == slot and i > pos and i < read_span[st][0]]
        assert not later_prev, f"slot {slot} read after DMA of {st}"
    # the epilogue stages C in the slot of the tile's last stage: its first write follows a barrier
    # that follows every wave's reads of that stage
    for n, (a, b) in enumerate(spans):
        S = (tiles[n][4] + 63) // 64
        if S:
            first_w = next(i for i in range(a, b) if ev[i][0] == "ds_write_b64")
            last_r = read_span[(n, S - 1)][1]
            assert any(last_r < bi < first_w for bi in barriers), f"tile {n}: staging races operand reads"
    # ---- MFMAs and stores per tile
    for n, (a, b) in enumerate(spans):
        S = (tiles[n][4] + 63) // 64
        mf = [ev[i] for i in range(a, b) if ev[i][0] == "mfma"]
        assert len(mf) == 24 * S
        for s in range(S):
            blk = mf[24 * s:24 * s + 24]
            dsts = {e[1] for e in blk}
            assert len(dsts) == 24
            for e in blk:
                assert (e[4] == "0") == (s == 0) and (e[4] == "0" or e[4] == e[1])
        st_ev = [ev[i] for i in range(a, b) if ev[i][0] == "store"]
        assert len(st_ev) == GEN.E_STORES
        g, m0, n0, kb, klen = tiles[n]
        offs = sorted(e[1][0] for e in st_ev)
        sw = (128 * (wave & 1) * stride_cm + 192 * (wave >> 1)) * 2
        want = sorted(sw + (32 * i + 8 * k) * 2 * stride_cm + 128 * p for i in range(4) for k in range(4)
                      for p in range(3))
        assert offs == want
        for e in st_ev:
            base, nrec, _, _ = e[2]
            assert base == OUT + 2 * (m0 * stride_cm + n0) and nrec == ((OUT_M - m0) * stride_cm - n0) * 2
            assert e[1][1] == _op("gb")
    assert state["np"] == 0 and state["nis"] == 0
    return ev


def _opidx(name):
    return [n for n, _ in GEN.OPERANDS].index(name)


def _op(name):
    return "%" + str(_opidx(name))


def _tiles(klens, seed=0):
    rng = np.random.default_rng(seed)
    out, kb = [], 0
    for n, k in enumerate(klens):
        out.append((n % 7, 256 * int(rng.integers(0, 11)), 384 * int(rng.integers(0, 15)), kb, int(k)))
        kb += int(k)
    return out


CASES = [
    [1], [64], [65], [128], [129], [200], [0], [0, 0], [1000],
    [64, 64, 64], [1, 1, 1, 1], [130, 0, 1, 63, 64, 65], [0, 500, 0, 7, 300],
    [4096, 4096, 4096], [127, 129, 191, 192, 193], [2, 200, 2, 200, 2],
]


@pytest.mark.parametrize("klens", CASES, ids=[f"case{i}" for i in range(len(CASES))])
def test_wide_pipeline_program(klens):
    _check(_tiles(klens, seed=len(klens)))


def test_wide_pipeline_random_sequences():
    rng = np.random.default_rng(7)
    for trial in range(40):
        n = int(rng.integers(1, 9))
        klens = [int(x) for x in rng.choice([0, 1, 31, 63, 64, 65, 127, 128, 129, 190, 320, 777], size=n)]
        _check(_tiles(klens, seed=trial), wave=trial % 4)


def test_waves_take_the_same_path():
    tiles = _tiles([130, 0, 1, 63, 64, 65, 300], seed=3)
    seqs = []
    for w in range(4):
        ev, _, _ = _run_tiles(tiles, w)
        seqs.append([e[0] for e in ev if e[0] in ("barrier", "mfma", "dma", "store", "read")])
    assert all(s == seqs[0] for s in seqs)


# ----------------------------------------------------------------------------- per-lane maps

def _swz_l(t):
    return (t & 7) << 1


def _swz_r(t):
    return ((t >> 1) & 3) << 1


def _lane_reads(w, width, lane_base_fn):
    """(lane, read k) -> (token, logical chunk, half) of the LDS bytes a transposed read touches."""
    out = {}
    for lane in range(64):
        for k, dt in enumerate((0, 8, 32, 40)):
            out[(lane, k)] = lane_base_fn(lane, dt)
    return out


def test_operand_reads_match_dma_placement_and_layout():
    """For every lane and read, the physical LDS address it reads holds (token, logical column
    chunk, half) = the 32x32x64 operand element the MFMA needs: row l % 32 of the block, tokens
    16 h + 0..15 in bytes 0-15 and 32 + 16 h + 0..15 in bytes 16-31 (h = l / 32)."""
    for side, width, swz, nblk in (("lhs", 256, _swz_l, 4), ("rhs", 384, _swz_r, 6)):
        for wv in range(2):   # wm for LHS, wn for RHS
            for blk in range(nblk):
                for lane in range(64):
                    g16, t16 = lane >> 4, lane & 15
                    cb, hh = g16 & 1, g16 >> 1
                    tb0, hb = 16 * hh + (t16 >> 1), t16 & 1
                    first = (8 * wv if side == "lhs" else 12 * wv) + 2 * blk
                    base = tb0 * width + 16 * ((first + cb) ^ swz(tb0)) + 8 * hb
                    for dt in (0, 8, 32, 40):
                        addr = base + dt * width
                        t = addr // width
                        pc = (addr % width) // 16
                        logical = pc ^ swz(t)   # the DMA stored logical chunk pc ^ swz(t) at pc
                        assert t == tb0 + dt and logical == first + cb and (addr % 16) // 8 == hb
                    # the tr_b8 read of the 16-lane group gives lane l column 16 cb + l % 16 of the
                    # block: operand row l % 32
                    assert 16 * cb + (lane % 16) == lane % 32


def test_operand_reads_conflict_free():
    for width, swz, first_fn in ((256, _swz_l, lambda wv, b: 8 * wv + 2 * b), (384, _swz_r, lambda wv, b: 12 * wv + 2 * b)):
        for wv in range(2):
            for blk in range(4 if width == 256 else 6):
                for dt in (0, 8, 32, 40):
                    for half in range(2):
                        pairs = set()
                        for lane in range(32 * half, 32 * half + 32):
                            g16, t16 = lane >> 4, lane & 15
                            cb, hh = g16 & 1, g16 >> 1
                            tb0, hb = 16 * hh + (t16 >> 1), t16 & 1
                            addr = (tb0 + dt) * width + 16 * ((first_fn(wv, blk) + cb) ^ swz(tb0)) + 8 * hb
                            pairs.add((addr // 8) % 32)
                        assert len(pairs) == 32


def test_dma_fills_each_slot_byte_once():
    stride_l, stride_r = 2880, 5760
    for width, n_inst, stride, swz in ((256, 16, stride_l, _swz_l), (384, 24, stride_r, _swz_r)):
        seen = {}
        for w in range(4):
            for j in range(n_inst // 4):
                i = w + 4 * j
                for lane in range(64):
                    q = 64 * i + lane
                    row, pc = q // (width // 16), q % (width // 16)
                    lds = 1024 * i + 16 * lane
                    assert lds == row * width + 16 * pc
                    if width == 256:
                        rowl, pcl = 4 * w + (lane >> 4), lane & 15
                        voff = rowl * stride + 16 * (pcl ^ swz(rowl)) + 16 * j * stride
                    else:
                        voff = row * stride + 16 * (pc ^ swz(row))
                    seen[lds] = voff
                    assert voff == row * stride + 16 * (pc ^ swz(row))
        assert sorted(seen) == list(range(0, 64 * width, 16))


def test_epilogue_staging_and_store_coverage():
    """Writes (row l % 32, chunk 4 jj + g, half l / 32) and read-backs (row 8 k + l / 8, chunk
    l % 8) address the same swizzled layout, each 16-byte chunk once, conflict-free (16 lanes per
    8-byte write cycle, 8 lanes per 16-byte read cycle); the stores then cover the 32 x 64 piece."""
    def phys(r, c):
        return r * 128 + 16 * (c ^ ((r >> 1) & 7))
    writes = {}
    for jj in range(2):
        for g in range(4):
            for lane in range(64):
                rl, hl = lane & 31, lane >> 5
                ew_base, ew_s = rl * 128 + 8 * hl, (rl >> 1) & 7
                addr = ew_base + (((4 * jj + g) ^ ew_s) << 4)
                assert addr == phys(rl, 4 * jj + g) + 8 * hl
                writes[addr] = (rl, 32 * jj + 8 * g + 4 * hl)     # row, first column of 4
            for q in range(4):
                banks = {((((lane & 31) * 128 + ((((4 * jj + g) ^ (((lane & 31) >> 1) & 7)) << 4)) + 8 * (lane >> 5)) // 8) % 32)
                         for lane in range(16 * q, 16 * q + 16)}
                assert len(banks) == 16
    assert len(writes) == 32 * 16
    cover = set()
    for k in range(4):
        for lane in range(64):
            rr, rc, rs = lane >> 3, lane & 7, ((lane >> 3) >> 1) & 7
            rb = (rr * 128 + 16 * (rc ^ rs)) if k % 2 == 0 else ((8 + rr) * 128 + 16 * (rc ^ (rs ^ 4)))
            addr = rb + (2048 if k >= 2 else 0)
            r = 8 * k + rr
            assert addr == phys(r, rc)
            assert writes[addr] == (r, 8 * rc) and writes[addr + 8] == (r, 8 * rc + 4)
            cover.add((r, rc))
        for q in range(8):
            chunks = {(((8 * k + (lane >> 3)) * 128 + 16 * ((lane & 7) ^ (((8 * k + (lane >> 3)) >> 1) & 7))) // 16) % 8
                      for lane in range(8 * q, 8 * q + 8)}
            assert len(chunks) == 8
    assert cover == {(r, c) for r in range(32) for c in range(8)}
