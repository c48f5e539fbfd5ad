"""CPU checks of the wide-tile wgrad kernels' generated assembly (ggemm-asm_amd/csrc/gen_vark_wide.py,
vark_wide.h; both tile shapes, 256 x 384 and 320 x 320), before any GPU launch.

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
  * issue BM x BN MFMAs per stage covering the blocks once (zero accumulator input in a tile's
    first stage), each after the LDS reads of its operands completed (in-order lgkmcnt), and the C
    stores of every epilogue pass, whose row/column offsets cover the wave's quadrant;
  * take the same branches and barriers in every wave.
The MXFP8 configuration also issues one e8m0 row per wave and stage (checked like the operand
rows), and every scaled MFMA must find, in the register half its op_sel_hi picks, the completed
scale read of its own block and stage.
Per-lane address maps (operand reads, LDS-DMA placement, epilogue staging, MX scale rows and the
epilogue bases the MX statement forms from the lane id) are checked against the 32x32x64 operand
layout and for LDS bank conflicts.
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


def _program(cfg):
    g = GEN.Gen(cfg)
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


CFGS = {c.name: c for c in GEN.CONFIGS}
PROGS = {name: _program(c) for name, c in CFGS.items()}


def _s32(x):
    x &= M32
    return x - (1 << 32) if x & 0x80000000 else x


class Block:
    """Runs the per-tile statement for one wave with given operand values."""

    def __init__(self, cfg, ops, events, scal, prog=None):
        self.cfg = cfg
        self.prog, self.labels = prog or PROGS[cfg.name]
        self.ops = ops          # operand name -> value (SGPR operands) / name (VGPR operands)
        self.ev = events
        self.s = scal           # persistent scalar temporaries (s56..s88), as on the GPU
        self.scc = 0
        self.v = {}             # symbolic VGPR temporaries

    def val(self, a):
        if a.startswith("%"):
            name = self.cfg.operands[int(a[1:])][0]
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
            name = self.cfg.operands[int(a[1:])][0]
            assert self.cfg.operands[int(a[1:])][1] == "+s", f"write to input operand {name}"
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
        PROG, LABELS = self.prog, self.labels
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
            elif op == "s_bitcmp1_b32":
                self.scc = (self.val(a[0]) >> int(a[1])) & 1
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
            elif op == "buffer_load_dwordx4" and a[-1].endswith("lds"):
                voff = self.v[a[0]] if a[0] in self.v and not a[0].startswith("%") else (0, a[0])
                self.ev.append(("dma", self.s["m0"], self.rsrc(a[1]), voff, a[-1]))
            elif op == "buffer_load_dwordx4":      # old values of an accumulated C, into VGPRs
                self.ev.append(("oload", self.v[a[1]], self.rsrc(a[2]), a[0]))
            elif op == "buffer_store_dwordx4":
                self.ev.append(("store", self.v[a[1]], self.rsrc(a[2]), a[0]))
            elif op == "ds_read_b64_tr_b8":
                reg, mod = a[1].split()
                base = self.v[reg]
                off = int(mod.split(":")[1])
                self.ev.append(("read", base, off, a[0]))
            elif op == "v_mfma_f32_32x32x64_f8f6f4":
                self.ev.append(("mfma", a[0], a[1], a[2], a[3].split()[0]))
            elif op == "v_mfma_scale_f32_32x32x64_f8f6f4":
                hi = re.search(r"op_sel_hi:\[(\d),(\d),(\d)\]", ",".join(a[5:])).groups()
                assert re.search(r"\bcbsz:1\b", ",".join(a[5:])) and "op_sel:" not in ",".join(a[5:])
                self.ev.append(("mfma", a[0], a[1], a[2], a[3], a[4], a[5].split()[0], (int(hi[0]), int(hi[1]))))
            elif op in ("ds_read_u8", "ds_read_u8_d16", "ds_read_u8_d16_hi"):
                reg, mod = a[1].split()
                # register halves written: (half, holds the byte) -- a full load zero-fills bits 16-31
                halves = {"ds_read_u8": ((0, True), (1, False)), "ds_read_u8_d16": ((0, True),),
                          "ds_read_u8_d16_hi": ((1, True),)}[op]
                self.ev.append(("sread", self.v[reg], int(mod.split(":")[1]), a[0], halves))
            elif op in ("ds_write_b64", "ds_write_b128", "ds_read_b128"):
                self.ev.append((op, a))
            elif op == "v_add_f32":          # fp32 accumulation: the old value added to the product
                self.ev.append(("vadd", a[0], a[1], a[2]))
            elif op.startswith("v_"):
                pass
            else:
                raise AssertionError(f"interpreter lacks {op}")
        return self


LHS, RHS, OUT = 0x7F0000000000, 0x7E0000000000, 0x7D0000000000
LSC, RSC = 0x7C0000000000, 0x7B0000000000       # MX e8m0 scales
STRIDE_LSC, STRIDE_RSC = 2896, 5776             # their row strides (at least the width, 16-aligned)


def _cb(cfg):
    """Bytes per C element."""
    return 2 if cfg.out == "bf16" else 4


def _run_tiles(cfg, tiles, wave, stride_l=2880, stride_r=5760, stride_cm=5760, OUT_M=2880, prog=None):
    """tiles: list of (g, m0, n0, kb, klen). Returns (events, per-tile event slices, final state)."""
    ev = []
    scal = {f"s{r}": 0 for r in cfg.sgpr_clobber}
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
                   cT_lo=(OUT + _cb(cfg) * (m0 * stride_cm + n0)) & M32,
                   cT_hi=(OUT + _cb(cfg) * (m0 * stride_cm + n0)) >> 32,
                   crecT=((OUT_M - m0) * stride_cm - n0) * _cb(cfg),
                   stride_l=stride_l, stride_r=stride_r, cm2=2 * stride_cm, alpha=0x3F800000,
                   sw_epi=(32 * cfg.bm * (wave & 1) * stride_cm + 32 * cfg.bn * (wave >> 1)) * _cb(cfg))
        if cfg.mx:
            side = wave >> 1
            base_sc, st_sc = (RSC, STRIDE_RSC) if side else (LSC, STRIDE_LSC)
            sct = base_sc + (kb >> 5) * st_sc + (n0 if side else m0)
            scn = base_sc + (N[3] >> 5) * st_sc + (N[2] if side else N[1])
            ops.update(scT_lo=sct & M32, scT_hi=sct >> 32, scN_lo=scn & M32, scN_hi=scn >> 32, stride_sc=st_sc,
                       scrd=(1024 + 160 * ((wave >> 1) - (wave & 1))) & M32, scw=GEN.SCALE_OFF + 1024 * side)
        start = len(ev)
        Block(cfg, ops, ev, scal, prog).run()
        spans.append((start, len(ev)))
        for k in state:
            state[k] = ops[k]
        state["c0"] = (state["c0"] + (klen + 63) // 64) % 3
    return ev, spans, state


def _check(cfg, tiles, wave=0, stride_l=2880, stride_r=5760, stride_cm=5760, OUT_M=2880, prog=None):
    ev, spans, state = _run_tiles(cfg, tiles, wave, stride_l, stride_r, stride_cm, OUT_M, prog)
    op = lambda name: "%" + str([n for n, _ in cfg.operands].index(name))
    L = cfg.loads
    stages = [(n, s) for n, t in enumerate(tiles) for s in range((t[4] + 63) // 64)]
    slot_of = {st: k % 3 for k, st in enumerate(stages)}
    # ---- DMA: one group of nl LHS + nr RHS loads per stage, in stage order
    dmas = [(i, e) for i, e in enumerate(ev) if e[0] == "dma"]
    assert len(dmas) == L * len(stages)
    issue_pos = {}
    for k, (n, s) in enumerate(stages):
        g, m0, n0, kb, klen = tiles[n]
        grp = dmas[L * k:L * k + L]
        issue_pos[(n, s)] = (grp[0][0], grp[-1][0])
        rv = min(64, klen - 64 * s)
        for j, (_, e) in enumerate(grp):
            _, m0v, (base, nrec, stride_bits, w3), voff, _ = e
            assert stride_bits == 0 and w3 == GEN.WORD3
            assert m0v + 1024 <= GEN.DMA_LDS_LIMIT          # LDS-DMA destinations below 128 KiB
            if j < cfg.nl:
                assert base == LHS + (kb + 64 * s) * stride_l + m0
                assert nrec == rv * stride_l - m0
                assert m0v == slot_of[(n, s)] * cfg.slot + 1024 * wave + 4096 * j
                assert voff == (0, op(f"voffL{j}"))
            elif j == cfg.nl + cfg.nr:
                # MX: the e8m0 rows of this wave's side (wave / 2) for the stage's two token blocks
                side = wave >> 1
                base_sc, st_sc = (RSC, STRIDE_RSC) if side else (LSC, STRIDE_LSC)
                assert base == base_sc + ((kb + 64 * s) >> 5) * st_sc + (n0 if side else m0)
                assert nrec == ((rv + 31) // 32 - 1) * st_sc + 320
                assert m0v == GEN.SCALE_OFF + ((slot_of[(n, s)] * cfg.slot) >> 4) + 1024 * side
                assert voff == (0, op("vsc"))
            else:
                jj = j - cfg.nl
                assert base == RHS + (kb + 64 * s) * stride_r + n0
                assert nrec == rv * stride_r - n0
                assert m0v == slot_of[(n, s)] * cfg.slot + cfg.rhs_off + 1024 * wave + 4096 * jj
                assert voff == (0, op(f"voffR{jj}"))
    # ---- reads: groups of 4 (bm + bn) in compute order, from the stage's slot
    R = 4 * (cfg.bm + cfg.bn)
    reads = [(i, e) for i, e in enumerate(ev) if e[0] == "read"]
    assert len(reads) == R * len(stages)
    read_span = {}
    want = []
    for side, nb, pitch in (("am", cfg.bm, cfg.tm), ("bn", cfg.bn, cfg.tn)):
        for b in range(nb):
            base, extra = cfg.read_base(side, b)
            want += [(base, extra + dt * pitch) for dt in GEN.TOK_OFFS]
    for k, st in enumerate(stages):
        grp = reads[R * k:R * k + R]
        read_span[st] = (grp[0][0], grp[-1][0])
        names = []
        for _, (_, (slot_off, name), off, dst) in grp:
            assert slot_off == slot_of[st] * cfg.slot, (st, slot_off)
            names.append((name, off))
        assert sorted(names) == sorted(want)
    # ---- completion model: in-order vmcnt, barriers
    issued = []            # event index of each vector-memory op, in order
    done_at = {}           # op index -> event index where it is known complete
    barriers = [i for i, e in enumerate(ev) if e[0] == "barrier"]
    for i, e in enumerate(ev):
        if e[0] in ("dma", "store", "oload"):
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
    # ---- operand data: every MFMA's A and B registers (and MX scale registers) hold completed reads
    # (in-order lgkmcnt); registers are tracked in 16-bit halves. No LDS load is issued into a
    # register another LDS load still in flight writes (a 16-bit load does not keep the other
    # half's value if the two overlap)
    def regs(r):
        m = re.fullmatch(r"v\[(\d+):(\d+)\]", r)
        return {(x, h) for x in range(int(m.group(1)), int(m.group(2)) + 1) for h in (0, 1)}
    pending = []           # (register halves written) of issued, not known complete LDS reads
    last_w = {}            # register half -> (slot value, base, offset) of the last scale read into it
    mfma_k = 0
    blk_of = {cfg.acc_range(i, j): (i, j) for i in range(cfg.bm) for j in range(cfg.bn)}
    def whole(hs):
        return {x for x, _ in hs}

    def issue_load(hs):
        assert not any(whole(hs) & whole(p) for p in pending), "two LDS loads in flight to one register"
        pending.append(hs)
    for e in ev:
        if e[0] == "read":
            issue_load(regs(e[3]))
        elif e[0] == "sread":
            r = int(e[3][1:])
            issue_load({(r, h) for h, _ in e[4]})
            for h, data in e[4]:
                last_w[(r, h)] = (e[1][0], e[1][1], e[2]) if data else ("zero", e[1][1], e[2])
        elif e[0] in ("ds_write_b64", "ds_write_b128"):
            pending.append(set())
        elif e[0] == "ds_read_b128":
            issue_load(regs(e[1][0]))
        elif e[0] == "lgkmcnt":
            pending = pending[len(pending) - e[1]:] if e[1] < len(pending) else pending
        elif e[0] == "mfma":
            need = regs(e[2]) | regs(e[3])
            if cfg.mx:
                (i, j), st = blk_of[e[1]], stages[mfma_k // (cfg.bm * cfg.bn)]
                ra, ha = cfg.scale_reg("bn", j)
                rb, hb = cfg.scale_reg("am", i)
                assert (e[5], e[6], e[7]) == (f"v{ra}", f"v{rb}", (ha, hb)), e
                sslot = (slot_of[st] * cfg.slot) >> 4
                scrd = (1024 + 160 * ((wave >> 1) - (wave & 1))) & M32
                assert last_w.get((rb, hb)) == (sslot, op("vscb"), 32 * i), f"MFMA {e}: LHS scale of {st}"
                assert last_w.get((ra, ha)) == ((sslot + scrd) & M32, op("vscb"), 32 * j), f"MFMA {e}: RHS scale"
                need |= {(ra, ha), (rb, hb)}
            mfma_k += 1
            assert not any(need & p for p in pending), f"MFMA {e} reads registers of a pending LDS read"
        elif e[0] == "store":
            assert not any(regs(e[3]) & p for p in pending), "store of pending LDS data"
    # ---- slot reuse: a DMA into a slot follows a barrier that follows every read of the previous
    # stage in that slot and every epilogue staging access there
    epi_slot_events = []
    for n, (a, b) in enumerate(spans):
        if (tiles[n][4] + 63) // 64 > 0:
            last = (n, (tiles[n][4] + 63) // 64 - 1)
            for i in range(a, b):
                if ev[i][0] in ("ds_write_b64", "ds_write_b128", "ds_read_b128"):
                    epi_slot_events.append((i, slot_of[last]))
    uses = sorted([(read_span[st][1], slot_of[st]) for st in stages] + epi_slot_events)
    for st in stages:
        pos = issue_pos[st][0]
        slot = slot_of[st]
        prior = [i for i, sl in uses if sl == slot and i < pos]
        if prior:
            assert any(max(prior) < bi < pos for bi in barriers), f"DMA of {st} into slot {slot} races a reader"
        later_prev = [i for i, sl in uses if sl == slot and pos < i < read_span[st][0]]
        assert not later_prev, f"slot {slot} read after DMA of {st}"
    # the epilogue stages C in the slot of the tile's last stage: its first write follows a barrier
    # that follows every wave's reads of that stage
    for n, (a, b) in enumerate(spans):
        S = (tiles[n][4] + 63) // 64
        if S:
            first_w = next(i for i in range(a, b) if ev[i][0] in ("ds_write_b64", "ds_write_b128"))
            last_r = read_span[(n, S - 1)][1]
            assert any(last_r < bi < first_w for bi in barriers), f"tile {n}: staging races operand reads"
    # ---- MFMAs and stores per tile
    nblk = cfg.bm * cfg.bn
    for n, (a, b) in enumerate(spans):
        S = (tiles[n][4] + 63) // 64
        mf = [ev[i] for i in range(a, b) if ev[i][0] == "mfma"]
        assert len(mf) == nblk * S
        for s in range(S):
            blk = mf[nblk * s:nblk * s + nblk]
            assert len({e[1] for e in blk}) == nblk
            for e in blk:
                assert (e[4] == "0") == (s == 0) and (e[4] == "0" or e[4] == e[1])
        st_ev = [(i, ev[i]) for i in range(a, b) if ev[i][0] == "store"]
        g, m0, n0, kb, klen = tiles[n]
        cbytes = _cb(cfg)
        sw = (32 * cfg.bm * (wave & 1) * stride_cm + 32 * cfg.bn * (wave >> 1)) * cbytes
        want_st = []
        if cfg.out == "bf16":
            # line-aligned pairs per wave half; with an odd block count the shared line's rows 0-15
            # (left half) or 16-31 (right half), from block bn - 1 / -1 of the wave's columns
            wn = wave >> 1
            gb = cfg.lane_regs.get("gb") or op("gb")
            for i in range(cfg.bm):
                if cfg.joint:
                    j0 = cfg.bn - 1 if wn == 0 else -1
                    for row, _, _ in GEN.Gen.joint_stores(wn):
                        want_st.append((sw + (32 * i + row) * 2 * stride_cm + 64 * j0, gb))
                for blocks in (cfg.pairs_wn1 if wn else cfg.pairs):
                    for row, _, _ in GEN.Gen.PAIR_STORES:
                        want_st.append((sw + (32 * i + row) * 2 * stride_cm + 64 * blocks[0], gb))
        elif not (cfg.out == "f32acc" and S == 0):
            for i in range(cfg.bm):
                for j in range(cfg.bn):
                    for k in range(4):
                        want_st.append((sw + (32 * i + 8 * k) * 4 * stride_cm + 128 * j, op("fgb")))
        assert sorted((e[1][0], e[1][1]) for _, e in st_ev) == sorted(want_st)
        for _, e in st_ev:
            base, nrec, _, _ = e[2]
            assert base == OUT + cbytes * (m0 * stride_cm + n0) and nrec == ((OUT_M - m0) * stride_cm - n0) * cbytes
        if cfg.out == "f32acc" and S:
            # every store follows the completed load of the old values at its offset
            ol = [(i, ev[i]) for i in range(a, b) if ev[i][0] == "oload"]
            assert sorted(e[1] for _, e in ol) == sorted(e[1] for _, e in st_ev)
            for si, se in st_ev:
                li = max(i for i, le in ol if le[1] == se[1] and i < si)
                assert li in done_at and done_at[li] < si, "store before its old values arrived"
            # register data flow: each stored register was last written by a v_add_f32 whose old-value
            # operand was last written by the completed load of that store's offset, same position
            # in the 16-byte chunk; accumulator registers reused as old-value buffers are loaded only
            # after their block's last read (its v_mul_f32s precede every load into them here)
            writer = {}
            for idx in range(a, b):
                e = ev[idx]
                if e[0] == "oload":
                    lo, hi = (int(x) for x in re.fullmatch(r"v\[(\d+):(\d+)\]", e[3]).groups())
                    for r in range(lo, hi + 1):
                        writer[r] = ("oload", idx, e[1], r - lo)
                elif e[0] == "ds_read_b128":
                    lo, hi = (int(x) for x in re.fullmatch(r"v\[(\d+):(\d+)\]", e[1][0]).groups())
                    for r in range(lo, hi + 1):
                        writer[r] = ("lds", idx)
                elif e[0] == "vadd":
                    d, s0, s1 = (int(x[1:]) for x in e[1:4])
                    assert d == s0 and writer.get(d, ("",))[0] == "lds", e
                    src = writer.get(s1)
                    assert src and src[0] == "oload", f"old-value operand v{s1} not from a load: {src}"
                    assert src[1] in done_at and done_at[src[1]] < idx, "add before its old value arrived"
                    writer[d] = ("vadd", idx, src[2], src[3])
                elif e[0] == "store":
                    lo, hi = (int(x) for x in re.fullmatch(r"v\[(\d+):(\d+)\]", e[3]).groups())
                    for r in range(lo, hi + 1):
                        w = writer.get(r)
                        assert w and w[0] == "vadd" and w[2] == e[1] and w[3] == r - lo, (e, w)
    assert state["np"] == 0 and state["nis"] == 0
    return ev


def _tiles(cfg, klens, seed=0):
    rng = np.random.default_rng(seed)
    out, kb = [], 0
    for n, k in enumerate(klens):
        out.append((n % 7, cfg.tm * int(rng.integers(0, 9)), cfg.tn * int(rng.integers(0, 15)), kb, int(k)))
        kb += int(k)
    return out


CASES = [
    [1], [64], [65], [128], [129], [200], [0], [0, 0], [1000],
    [64, 64, 64], [1, 1, 1, 1], [130, 0, 1, 63, 64, 65], [0, 500, 0, 7, 300],
    [4096, 4096, 4096], [127, 129, 191, 192, 193], [2, 200, 2, 200, 2],
]


@pytest.mark.parametrize("cfg", list(CFGS))
@pytest.mark.parametrize("klens", CASES, ids=[f"case{i}" for i in range(len(CASES))])
def test_wide_pipeline_program(cfg, klens):
    c = CFGS[cfg]
    _check(c, _tiles(c, klens, seed=len(klens)), stride_cm=5760 if cfg == "256x384" else 5760)


@pytest.mark.parametrize("cfg", list(CFGS))
def test_wide_pipeline_random_sequences(cfg):
    c = CFGS[cfg]
    rng = np.random.default_rng(7)
    for trial in range(40):
        n = int(rng.integers(1, 9))
        klens = [int(x) for x in rng.choice([0, 1, 31, 63, 64, 65, 127, 128, 129, 190, 320, 777], size=n)]
        _check(c, _tiles(c, klens, seed=trial), wave=trial % 4)


@pytest.mark.parametrize("cfg", list(CFGS))
def test_waves_take_the_same_path(cfg):
    c = CFGS[cfg]
    tiles = _tiles(c, [130, 0, 1, 63, 64, 65, 300], seed=3)
    seqs = []
    for w in range(4):
        ev, _, _ = _run_tiles(c, tiles, w)
        seqs.append([e[0] for e in ev if e[0] in ("barrier", "mfma", "dma", "store", "read")])
    assert all(sq == seqs[0] for sq in seqs)


def test_generated_include_is_current():
    """vark_wide_asm.inc in the tree is what the generator writes (the build regenerates it)."""
    text, _ = GEN.render()
    assert open(GEN.OUT).read() == text


def test_asm_writes_only_clobbered_registers():
    for c in GEN.CONFIGS:
        g = GEN.Gen(c)
        g.tile()
        for line in g.lines:
            for m in re.finditer(r"\b([sva])\[?(\d+)(?::(\d+)\])?", line):
                k, lo = m.group(1), int(m.group(2))
                hi = int(m.group(3)) if m.group(3) else lo
                if k == "s":
                    assert c.sgpr_clobber[0] <= lo and hi <= c.sgpr_clobber[-1], line
                elif k == "v":
                    assert c.vgpr_clobber[0] <= lo and hi <= 255, line
                else:
                    assert hi <= 255, line


# ----------------------------------------------------------------------------- per-lane maps
# Restated from vark_wide.h's set-up (amb / bnb / voff / epilogue bases) and checked for layout
# and conflicts.

def _lane(lane):
    g16, t16 = lane >> 4, lane & 15
    return g16 & 1, 16 * (g16 >> 1) + (t16 >> 1), t16 & 1      # cb, tb0, hb


def _block_base(cfg, side, wv, b, lane):
    """Byte offset (slot-relative) of block b's first transposed read, as vark_wide.h forms it."""
    cb, tb0, hb = _lane(lane)
    pitch, nb = (cfg.tm, cfg.bm) if side == "am" else (cfg.tn, cfg.bn)
    off = 0 if side == "am" else cfg.rhs_off
    swz = GEN.swizzle(pitch)
    return off + tb0 * pitch + 16 * ((2 * nb * wv + 2 * b + cb) ^ swz(tb0)) + 8 * hb


@pytest.mark.parametrize("cfg", list(CFGS))
def test_operand_reads_match_dma_placement_and_layout(cfg):
    """For every lane and read, the physical LDS address it reads holds (token, logical column
    chunk, half) = the 32x32x64 operand element the MFMA needs: row l % 32 of the block, tokens
    16 h + 0..15 in bytes 0-15 and 32 + 16 h + 0..15 in bytes 16-31 (h = l / 32). With parity
    bases, block b's address is base[b & 1] + 32 b as the assembly forms it."""
    c = CFGS[cfg]
    for side, nb, pitch in (("am", c.bm, c.tm), ("bn", c.bn, c.tn)):
        swz = GEN.swizzle(pitch)
        off = 0 if side == "am" else c.rhs_off
        for wv in range(2):
            for b in range(nb):
                for lane in range(64):
                    cb, tb0, hb = _lane(lane)
                    base = _block_base(c, side, wv, b, lane)
                    if c.parity_bases:
                        pb = _block_base(c, side, wv, b & 1, lane) - 32 * (b & 1)
                        assert pb + 32 * b == base
                    first = 2 * nb * wv + 2 * b
                    for dt in GEN.TOK_OFFS:
                        addr = base + dt * pitch - off
                        t, pc = addr // pitch, (addr % pitch) // 16
                        assert t == tb0 + dt and pc ^ swz(t) == first + cb and (addr % 16) // 8 == hb
                    assert 16 * cb + (lane % 16) == lane % 32


@pytest.mark.parametrize("cfg", list(CFGS))
def test_operand_reads_conflict_free(cfg):
    c = CFGS[cfg]
    for side, nb, pitch in (("am", c.bm, c.tm), ("bn", c.bn, c.tn)):
        for wv in range(2):
            for b in range(nb):
                for dt in GEN.TOK_OFFS:
                    for half in range(2):
                        pairs = {((_block_base(c, side, wv, b, lane) + dt * pitch) // 8) % 32
                                 for lane in range(32 * half, 32 * half + 32)}
                        assert len(pairs) == 32


@pytest.mark.parametrize("cfg", list(CFGS))
def test_dma_fills_each_slot_byte_once(cfg):
    c = CFGS[cfg]
    for pitch, n_inst, stride in ((c.tm, 4 * c.nl, 2880), (c.tn, 4 * c.nr, 5760)):
        swz = GEN.swizzle(pitch)
        seen = {}
        for w in range(4):
            for j in range(n_inst // 4):
                i = w + 4 * j
                for lane in range(64):
                    q = 64 * i + lane
                    row, pc = q // (pitch // 16), q % (pitch // 16)
                    lds = 1024 * i + 16 * lane
                    assert lds == row * pitch + 16 * pc
                    seen[lds] = row * stride + 16 * (pc ^ swz(row))
        assert sorted(seen) == list(range(0, 64 * pitch, 16))
        # the logical chunks of each row are each loaded once
        rows = {}
        for lds, voff in seen.items():
            rows.setdefault(voff // stride, []).append((voff % stride) // 16)
        assert all(sorted(v) == list(range(pitch // 16)) for v in rows.values())


def _phys(r, cc):
    return r * 128 + 16 * (cc ^ ((r >> 1) & 7))


def test_epilogue_staging_and_store_coverage():
    """Writes (row l % 32, chunk 4 jj + g, half l / 32) and read-backs (row 8 k + l / 8, chunk
    l % 8) address the same swizzled layout, each 16-byte chunk once, conflict-free (16 lanes per
    8-byte write cycle, 8 lanes per 16-byte read cycle); the stores then cover the 32 x 64 piece."""
    writes = {}
    for jj in range(2):
        for g in range(4):
            for lane in range(64):
                rl, hl = lane & 31, lane >> 5
                ew_base, ew_s = rl * 128 + 8 * hl, (rl >> 1) & 7
                addr = ew_base + (((4 * jj + g) ^ ew_s) << 4)
                assert addr == _phys(rl, 4 * jj + g) + 8 * hl
                writes[addr] = (rl, 32 * jj + 8 * g + 4 * hl)     # row, first column of 4
            for q in range(4):
                banks = {(((lane & 31) * 128 + ((((4 * jj + g) ^ (((lane & 31) >> 1) & 7)) << 4))
                           + 8 * (lane >> 5)) // 8) % 32 for lane in range(16 * q, 16 * q + 16)}
                assert len(banks) == 16
    assert len(writes) == 32 * 8 * 2
    cover = set()
    for k, (row, rb, off) in enumerate(GEN.Gen.PAIR_STORES):
        addrs = []
        for lane in range(64):
            rr, rc, rs = lane >> 3, lane & 7, ((lane >> 3) >> 1) & 7
            base = (rr * 128 + 16 * (rc ^ rs)) if rb == 0 else ((8 + rr) * 128 + 16 * (rc ^ (rs ^ 4)))
            r, cc = row + rr, rc
            addr = base + off
            assert addr == _phys(r, cc)
            assert writes[addr] == (r, 8 * cc) and writes[addr + 8] == (r, 8 * cc + 4)
            cover.add((r, cc))
            addrs.append(addr)
        for q in range(8):
            assert len({(a // 16) % 16 for a in addrs[8 * q:8 * q + 8]}) == 8   # 16-byte bank groups
    assert cover == {(r, cc) for r in range(32) for cc in range(8)}


@pytest.mark.parametrize("cfg", [n for n, c in CFGS.items() if c.out == "bf16" and c.joint])
def test_epilogue_joint_line(cfg):
    """The line two wave halves share: the left half writes its block bn - 1 into chunks 0-3 of the
    common region's rows, the right half its block 0 into chunks 4-7 (the pass's write addresses of
    jj = 0 / 1); after the barrier the left half reads rows 0-15 and the right half rows 16-31 with
    the pair read-back, so every row of the line -- columns 32 (bn - 1) .. 32 bn + 31 of the left
    half's frame, i.e. tile columns 32 bn - 32 .. 32 bn + 31 -- is stored whole, once, by one wave,
    at the column the store offset names (block bn - 1 for the left half, block -1 for the right)."""
    c = CFGS[cfg]
    region = {}
    for wn, jj, blk in ((0, 0, c.bn - 1), (1, 1, 0)):
        for g in range(4):
            for lane in range(64):
                rl, hl = lane & 31, lane >> 5
                addr = rl * 128 + 8 * hl + (((4 * jj + g) ^ ((rl >> 1) & 7)) << 4)
                col = 32 * c.bn * wn + 32 * blk + 8 * g + 4 * hl        # tile column of 4 values
                assert addr not in region
                region[addr] = (rl, col)
    stored = {}
    for wn in range(2):
        j0 = c.bn - 1 if wn == 0 else -1
        for row, rb, off in GEN.Gen.joint_stores(wn):
            for lane in range(64):
                rr, rc, rs = lane >> 3, lane & 7, ((lane >> 3) >> 1) & 7
                base = (rr * 128 + 16 * (rc ^ rs)) if rb == 0 else ((8 + rr) * 128 + 16 * (rc ^ (rs ^ 4)))
                r = row + rr
                gcol = 32 * c.bn * wn + 32 * j0 + 8 * rc          # where the store puts the chunk
                assert region[base + off] == (r, gcol) and region[base + off + 8] == (r, gcol + 4)
                assert (r, gcol) not in stored
                stored[(r, gcol)] = wn
    assert set(stored) == {(r, 32 * c.bn - 32 + 8 * q) for r in range(32) for q in range(8)}


def test_epilogue_f32_staging_and_store_coverage():
    """fp32 passes (one 32 x 32 block): lane (r = l % 32, h = l / 32) writes chunk 2 g + h of row r
    at fw_base + 32 (g ^ fw_s), the layout chunk c of row r at c ^ (((r >> 1) & 3) << 1); read-back k
    gives lane l row 8 k + l / 8, chunk l % 8 at frb + 1024 k. Each chunk written and read once,
    16-byte accesses conflict-free 8 lanes at a time, 8 lanes per whole 128-byte row."""
    def phys(r, cc):
        return r * 128 + 16 * (cc ^ (((r >> 1) & 3) << 1))
    writes = {}
    for g in range(4):
        addrs = []
        for lane in range(64):
            rl, hl = lane & 31, lane >> 5
            fw_base, fw_s = rl * 128 + 16 * hl, (rl >> 1) & 3
            addr = fw_base + 32 * (g ^ fw_s)
            assert addr == phys(rl, 2 * g + hl)
            writes[addr] = (rl, 8 * g + 4 * hl)          # row, first of 4 fp32 columns
            addrs.append(addr)
        for q in range(8):
            assert len({(a // 16) % 16 for a in addrs[8 * q:8 * q + 8]}) == 8
    assert len(writes) == 32 * 8
    cover = set()
    for k in range(4):
        addrs = []
        for lane in range(64):
            rr, rc = lane >> 3, lane & 7
            frb = rr * 128 + 16 * (rc ^ (((rr >> 1) & 3) << 1))
            addr = frb + 1024 * k
            r = 8 * k + rr
            assert addr == phys(r, rc) and writes[addr] == (r, 4 * rc)
            cover.add((r, rc))
            addrs.append(addr)
        for q in range(8):
            assert len({(a // 16) % 16 for a in addrs[8 * q:8 * q + 8]}) == 8
    assert cover == {(r, cc) for r in range(32) for cc in range(8)}


# ----------------------------------------------------------------------------- MXFP8 per-lane maps

MXC = CFGS["320x320_mx"]


def test_mx_scale_rows_reach_each_lane():
    """The scale slot as the four waves' LDS-DMA fills it (vark_wide.h: both waves of side v / 2
    carry that side's two rows, lane l < 40 chunk l % 20 of row l / 20 with vsc = (l / 20) stride +
    16 (l % 20) to scw + 16 l, the other lanes out of range), read as the statement reads it (vscb +
    32 b, RHS + scrd): every lane of every wave gets, for each m-block i / n-block j, the e8m0 byte
    of row l % 32 of that block in token block l / 32 -- the lane the scaled 32x32x64 MFMA takes the
    scale of (row l % 32, K-block l / 32) from, K-block 0 being the stage's tokens 0-31 (bytes 0-15
    of both lane halves). The two waves of a side write identical bytes, and all of it lies below
    128 KiB and inside the slot's 2.5 KiB."""
    rng = np.random.default_rng(11)
    for st_l, st_r, m0, n0, blk0 in ((2896, 5776, 320 * 3, 320 * 7, 5), (320, 320, 0, 0, 0)):
        lsc = rng.integers(0, 255, size=(blk0 + 2, st_l), dtype=np.uint8)
        rsc = rng.integers(0, 255, size=(blk0 + 2, st_r), dtype=np.uint8)
        for slot_idx in range(3):
            sbase = GEN.SCALE_OFF + ((slot_idx * MXC.slot) >> 4)
            lds = {}
            for v in range(4):
                side = v >> 1
                sc, st, col = (rsc, st_r, n0) if side else (lsc, st_l, m0)
                flat = sc.reshape(-1)
                nrec = 1 * st + 320                       # both blocks valid
                scw = GEN.SCALE_OFF + 1024 * side
                for lane in range(64):
                    vsc = (lane // 20) * st + 16 * (lane % 20) if lane < 40 else 0x80000000
                    data = flat[blk0 * st + col + vsc:][:16] if vsc + 16 <= nrec else np.zeros(16, np.uint8)
                    assert (vsc + 16 <= nrec) == (lane < 40)
                    dst = scw + ((slot_idx * MXC.slot) >> 4) + 16 * lane
                    assert sbase <= dst and dst + 16 <= sbase + GEN.SCALE_SLOT and dst + 16 <= GEN.DMA_LDS_LIMIT
                    for k in range(16):
                        assert lds.setdefault(dst + k, int(data[k])) == int(data[k])   # same bytes from both waves
            for w in range(4):
                wm, wn = w & 1, w >> 1
                scrd = 1024 + 160 * (wn - wm)
                for lane in range(64):
                    vscb = GEN.SCALE_OFF + 320 * (lane >> 5) + 160 * wm + (lane & 31)
                    kb, row = lane >> 5, lane & 31
                    for b in range(MXC.bm):
                        assert lds[sbase - GEN.SCALE_OFF + vscb + 32 * b] == lsc[blk0 + kb, m0 + 160 * wm + 32 * b + row]
                    for b in range(MXC.bn):
                        assert (lds[sbase - GEN.SCALE_OFF + vscb + scrd + 32 * b]
                                == rsc[blk0 + kb, n0 + 160 * wn + 32 * b + row])


def test_mx_scale_reads_conflict_free():
    """One scale read (ds_read_u8, 64 lanes): the 32 lanes of a half read 32 consecutive bytes of
    one row, so at most 4 lanes share a 4-byte bank word and no two lanes hit one bank in
    different words."""
    for w in range(4):
        wm, wn = w & 1, w >> 1
        for extra in [32 * b for b in range(5)] + [1024 + 160 * (wn - wm) + 32 * b for b in range(5)]:
            for half in range(2):
                addrs = [320 * (lane >> 5) + 160 * wm + (lane & 31) + extra for lane in range(32 * half, 32 * half + 32)]
                words = {}
                for a in addrs:
                    words.setdefault((a // 4) % 64, set()).add(a // 4)
                assert all(len(v) == 1 for v in words.values())


def _eval_lane_values(cfg, stride_cm):
    """Runs the statement's lane-id sequence (Gen.lane_values) for every lane."""
    g = GEN.Gen(cfg)
    g.lane_values()
    ops = {cfg.op["cm2"]: 2 * stride_cm}
    out = []
    for lane in range(64):
        v = {}

        def val(x):
            if x in ops:
                return ops[x]
            if x.startswith("v"):
                return v[x]
            return int(x, 0)
        for line in g.lines:
            op, _, rest = line.partition(" ")
            a = [t.strip() for t in rest.split(",")]
            if op == "v_mbcnt_lo_u32_b32":
                assert a[1:] == ["-1", "0"]
                v[a[0]] = min(lane, 32)
            elif op == "v_mbcnt_hi_u32_b32":
                assert a[1] == "-1"
                v[a[0]] = val(a[2]) + max(lane - 32, 0)
            elif op == "v_and_b32":
                v[a[0]] = val(a[1]) & val(a[2])
            elif op == "v_xor_b32":
                v[a[0]] = val(a[1]) ^ val(a[2])
            elif op == "v_lshrrev_b32":
                v[a[0]] = val(a[2]) >> val(a[1])
            elif op == "v_lshlrev_b32":
                v[a[0]] = (val(a[2]) << val(a[1])) & M32
            elif op == "v_lshl_add_u32":
                v[a[0]] = ((val(a[1]) << val(a[2])) + val(a[3])) & M32
            elif op == "v_bfe_u32":
                v[a[0]] = (val(a[1]) >> val(a[2])) & ((1 << val(a[3])) - 1)
            elif op == "v_add_u32":
                v[a[0]] = (val(a[1]) + val(a[2])) & M32
            elif op == "v_mul_lo_u32":
                v[a[0]] = (val(a[1]) * val(a[2])) & M32
            else:
                raise AssertionError(op)
        out.append({n: v[r] for n, r in cfg.lane_regs.items()})
    return out


@pytest.mark.parametrize("stride_cm", [5760, 2880, 320])
def test_mx_epilogue_lane_values(stride_cm):
    """The epilogue bases the MX statement forms from the lane id equal the values vark_wide.h
    passes the other configurations as operands."""
    got = _eval_lane_values(MXC, stride_cm)
    for lane in range(64):
        rl, hl = lane & 31, lane >> 5
        rr, rc = lane >> 3, lane & 7
        rs = (rr >> 1) & 7
        r1, c1 = lane >> 2, lane & 3
        want = dict(ew_base=rl * 128 + 8 * hl, ew_s=(rl >> 1) & 7, rb_even=rr * 128 + 16 * (rc ^ rs),
                    rb_odd=(8 + rr) * 128 + 16 * (rc ^ (rs ^ 4)), gb=(rr * stride_cm + 8 * rc) * 2)
        assert got[lane] == want, lane


def test_mx_lane_value_registers_are_free():
    """The registers the MX epilogue forms its bases (and temporaries) in lie in the operand
    registers, clear of the staging registers the bf16 epilogue uses (vop0 .. vop0 + 55) and of the
    accumulators."""
    regs = {int(r[1:]) for r in MXC.lane_regs.values()}
    g = GEN.Gen(MXC)
    g.lane_values()
    for line in g.lines:
        regs |= {int(m) for m in re.findall(r"\bv(\d+)\b", line.split(" ", 1)[1].split(",")[0])}
    assert min(regs) >= MXC.vop0 + 56 and max(regs) < MXC.vacc0


@pytest.mark.parametrize("cfg", [n for n, c in CFGS.items() if c.out == "bf16"])
def test_bf16_stores_whole_lines(cfg):
    """Every bf16 store writes 128-byte row pieces starting on a 128-byte boundary of the tile row
    (a C row starts on one at the MoE shapes): the pairs of each wave half and the joint pass's
    shared line; together they cover each wave's blocks once."""
    c = CFGS[cfg]
    for wn in range(2):
        starts = [2 * (32 * c.bn * wn + 32 * blocks[0]) for blocks in (c.pairs_wn1 if wn else c.pairs)]
        if c.joint:
            starts.append(2 * (32 * c.bn * wn + 32 * (c.bn - 1 if wn == 0 else -1)))
        assert all(x % 128 == 0 for x in starts), (wn, starts)
        got = sorted(j for blocks in (c.pairs_wn1 if wn else c.pairs) for j in blocks)
        got += [c.joint_block[wn]] if c.joint else []
        assert sorted(got) == list(range(c.bn))


@pytest.mark.parametrize("cfg", [n for n, c in CFGS.items() if c.out == "bf16" and c.joint])
@pytest.mark.parametrize("wave", range(4))
def test_epilogue_joint_region_ordering(cfg, wave):
    """The common region is written by one wave and read by another, so in each wave's program:
    an m-block's joint writes complete (lgkmcnt(0)) and a barrier follows before its joint reads;
    a buffer (m-block parity) is written again only after a barrier that follows this wave's reads
    of it -- the partner passes the same barriers, so its reads are done too."""
    c = CFGS[cfg]
    ev, spans, _ = _run_tiles(c, [(0, 0, 0, 0, 100)], wave)
    a, b = spans[0]
    v0 = c.vop0
    xw = {f"v{v0 + 70 + g}" for g in range(4)}
    xr = {f"v{v0 + 74 + k}" for k in range(2)}

    def off(arg):
        m = re.search(r"offset:(\d+)", arg)
        return int(m.group(1)) if m else 0
    seq = []
    for i in range(a, b):
        e = ev[i]
        if e[0] == "ds_write_b64" and e[1][0].split()[0] in xw:
            seq.append(("w", off(e[1][-1]) // 4096, i))
        elif e[0] == "ds_read_b128" and e[1][1].split()[0] in xr:
            seq.append(("r", (off(e[1][1]) % 8192) // 4096, i))
        elif e[0] in ("barrier", "lgkmcnt"):
            seq.append((e[0], e[1] if e[0] == "lgkmcnt" else None, i))
    writes = [x for x in seq if x[0] == "w"]
    reads = [x for x in seq if x[0] == "r"]
    assert len(writes) == 4 * c.bm and len(reads) == 2 * c.bm
    for blk in range(c.bm):
        w = writes[4 * blk:4 * blk + 4]
        r = reads[2 * blk:2 * blk + 2]
        assert {x[1] for x in w} == {blk % 2} and {x[1] for x in r} == {blk % 2}
        between = [x for x in seq if w[-1][2] < x[2] < r[0][2]]
        kinds = [x[0] for x in between]
        assert "barrier" in kinds and ("lgkmcnt", 0) in [(x[0], x[1]) for x in between[:kinds.index("barrier")]]
        if blk + 2 < c.bm:
            nxt = writes[4 * (blk + 2)]
            assert any(x[0] == "barrier" and r[-1][2] < x[2] < nxt[2] for x in seq)
