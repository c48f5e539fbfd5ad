#!/usr/bin/env python3
"""Writes vark_wide_asm.inc: the per-tile body of the wide-tile FP8 grouped wgrad kernels
(vark_wide.h), one gfx950 inline-assembly statement per tile configuration.

Why assembly: a wide output tile on four waves (one per SIMD) needs 384 (256 x 384) or 400
(320 x 320) fp32 accumulators per wave, 256 in AGPRs and the rest in VGPRs. The compiler gives
every MFMA of a kernel the same accumulator register class (at most 256 AGPRs), so it cannot build
these kernels without spilling; written out here, the accumulators sit in fixed registers for the
whole K loop.

One statement computes one tile of one group (the HIP code around it walks the schedule, see
vark_wide.h) and keeps the operand pipeline running across tiles:
  * the token axis in stages of 64: LDS holds three stage slots (64 rows of the tile's LHS bytes,
    then 64 rows of its RHS bytes, 40 KiB), filled by LDS-DMA (buffer_load_dwordx4 ... lds, 1 KiB
    per wave-instruction, 10 per wave and stage), bounded by the buffer's num_records so tokens
    past the group end read as zero;
  * an issue cursor walks this tile's stages, then the next tile's first two: at each stage's
    barrier the slot just released takes the cursor's next stage, so up to three stages are in
    flight; counted vmcnt waits use a per-wave model of outstanding vector-memory operations
    (in/out operands, so it survives between tiles);
  * per stage and wave BM x BN v_mfma_f32_32x32x64_f8f6f4 (BM LHS blocks x BN RHS blocks of 32;
    A = RHS e5m2 with cbsz 1, B = LHS e4m3), operands read with ds_read_b64_tr_b8 as the MFMAs
    release their registers, the barrier that publishes the next stage after the first row of
    MFMAs, the next stage's LDS-DMA one instruction per MFMA gap;
  * the epilogue scales by s_lhs * s_rhs, converts to bf16 (RNE), stages 32-row pieces through the
    freed slot (XOR swizzle, conflict-free) and stores whole row chunks non-temporally; rows past
    OUT_M fall outside the C buffer resource and are dropped.

Each configuration's operands (numbered as the asm statement in vark_wide.h passes them) are
listed by Config.operands; run this script to rewrite the include after changing it (build.py runs
it before every build).
"""
from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "vark_wide_asm.inc")

SLOTS = 3
WORD3 = 0x00020000           # raw buffer resource word 3 (32-bit data format)
KS = 64                      # tokens per stage
TOK_OFFS = (0, 8, 32, 40)    # token offsets of the four transposed reads of a 32x32x64 operand

# scalar temporaries (clobbered): buffer resources in aligned quads, then state
SGPR = dict(
    RL="s[56:59]", RL0="s56", RL1="s57", RL2="s58", RL3="s59",
    RR="s[60:63]", RR0="s60", RR1="s61", RR2="s62", RR3="s63",
    RC="s[64:67]", RC0="s64", RC1="s65", RC2="s66", RC3="s67",
    S="s68", K="s69", INT="s70", IDX="s71", REM="s72", LIM="s73",
    BL0="s74", BL1="s75", BR0="s76", BR1="s77", CM0="s78", CN0="s79",
    ISLOT="s80", CS="s81", NS="s82", T="s83", T2="s84", NEED="s85", LIMTOP="s86", EPI="s87", IB="s88",
    # MXFP8 only: the cursor's scale pointer, the scale resource, the read slot's scale offsets
    BS0="s89", BS1="s90", NSS="s91", RS="s[92:95]", RS0="s92", RS1="s93", RS2="s94", RS3="s95", NSSR="s96",
)
SGPR_CLOBBER = list(range(56, 89))
SGPR_CLOBBER_MX = list(range(56, 97))
# MXFP8: the e8m0 rows of a stage sit in a scale slot at SCALE_OFF + (stage slot offset >> 4): the
# LHS rows of token blocks 0 and 1 at +0 and +320, the RHS rows at +1024 and +1344. Every LDS-DMA
# destination of these kernels stays below 128 KiB, the range the operand slots have always used
# (the DMA's M0 offset is not exercised above it); the schedule tables, read with plain LDS reads,
# move above the scale slots.
SCALE_OFF = SLOTS * 40960
SCALE_SLOT = 40960 >> 4
DMA_LDS_LIMIT = 128 * 1024


def swizzle(pitch):
    """Chunk swizzle of a token row of `pitch` bytes (a function of the token index): the 8 tokens
    x 2 chunks x 2 halves a 32-lane half of a transposed read touches land in 32 distinct 8-byte
    bank pairs, and tokens t + 8, t + 32, t + 40 share t's swizzle."""
    if pitch == 256:
        return lambda t: (t & 7) << 1
    if pitch == 384:
        return lambda t: ((t >> 1) & 3) << 1
    if pitch == 320:
        return lambda t: ((t >> 2) & 1) << 1
    raise ValueError(pitch)


class Config:
    def __init__(self, tm, tn, out="bf16", mx=False):
        self.tm, self.tn = tm, tn
        self.out = out                                  # "bf16", "f32" (fp32 C) or "f32acc" (C += result)
        self.mx = mx                                    # MXFP8: e8m0 block scales, scaled MFMA
        assert not mx or (out == "bf16" and tm == tn == 320)
        self.name = f"{tm}x{tn}" + ("" if out == "bf16" else "_" + out) + ("_mx" if mx else "")
        self.bm, self.bn = tm // 64, tn // 64           # 32-wide blocks per wave (2 x 2 waves)
        self.rhs_off = KS * tm
        self.slot = KS * (tm + tn)
        self.nl = KS * tm // 1024 // 4                  # LHS / RHS LDS-DMA instructions per wave
        self.nr = KS * tn // 1024 // 4
        self.loads = self.nl + self.nr + (1 if mx else 0)   # MX: one scale row per wave
        nblk = self.bm * self.bn
        self.vacc0 = 256 - 16 * (nblk - 16)             # first VGPR accumulator
        # MX: the lane's e8m0 scale of each block of the stage, one register each (byte 0, read
        # with a full-register ds_read_u8). Two blocks cannot share a register through 16-bit
        # loads: on gfx950 a ds_read_u8_d16(_hi) zeroes the other half (measured on MI355X).
        if mx:
            self.scale_map = {**{("am", i): (i, 0) for i in range(self.bm)},
                              **{("bn", j): (self.bm + j, 0) for j in range(self.bn)}}
            self.nsl, self.nsr = self.bm, self.bn
        else:
            self.scale_map, self.nsl, self.nsr = {}, 0, 0
        self.vop0 = self.vacc0 - 8 * (self.bm + self.bn)   # operand tuples (even-aligned)
        self.vsc0 = self.vop0 - self.nsl - self.nsr        # MX scale registers below them
        # vt: read-address temporary; vt2: the epilogue's store offset (MX: the last scale
        # register, free by then -- the K loop never uses vt2)
        self.vt = f"v{self.vsc0 - (1 if mx else 2)}"
        self.vt2 = f"v{self.vop0 - 1}"
        self.vgpr_clobber = list(range(self.vsc0 - (1 if mx else 2), 256))
        # the bf16 epilogue's joint-pass addresses (four writes, two reads) in operand registers
        self.epi_x = self.vop0 + 70
        assert self.epi_x + 6 <= self.vacc0
        self.sgpr_clobber = SGPR_CLOBBER_MX if mx else SGPR_CLOBBER
        self.rb = 5 if mx else 4                        # LDS reads per operand block (MX: + its scale)
        # bf16 passes of two blocks (64 columns: one 128-byte C line per row). With an odd block count
        # the right-half waves (wn = 1) start half a line into the tile row: the left half pairs
        # blocks (0, 1), (2, 3), ..., the right half (1, 2), (3, 4), ..., and the line the two halves
        # share (left block bn - 1, right block 0) goes through a joint pass: both waves stage their
        # block in one LDS region, and after a barrier each stores half of its rows as whole lines.
        self.joint = self.bn % 2 == 1
        self.pairs = [(2 * q, 2 * q + 1) for q in range(self.bn // 2)]
        self.pairs_wn1 = [(2 * q + 1, 2 * q + 2) for q in range(self.bn // 2)] if self.joint else self.pairs
        self.joint_block = (self.bn - 1, 0)            # (left wave's block, right wave's block)
        if out == "bf16":
            self.e_stores = self.bm * (4 * len(self.pairs) + (2 if self.joint else 0))
        else:
            # fp32: one 32 x 32 block per pass, four 1 KiB stores (and, accumulating, four loads of
            # the old values); the counted waits saturate at vmcnt's 63
            self.e_stores = nblk * (8 if out == "f32acc" else 4)
        # read bases: one per block, or (320-byte rows, one-bit swizzle) two per side by parity
        self.parity_bases = tm == 320 and tn == 320
        ops = [("c0", "+s"), ("nis", "+s"), ("vmt", "+s"), ("q0", "+s"), ("q1", "+s"), ("q2", "+s"), ("np", "+s"),
               ("lds_base", "s"), ("w1k", "s"),
               ("bLT_lo", "s"), ("bLT_hi", "s"), ("bRT_lo", "s"), ("bRT_hi", "s"), ("klenT", "s"), ("m0T", "s"),
               ("n0T", "s"),
               ("bLN_lo", "s"), ("bLN_hi", "s"), ("bRN_lo", "s"), ("bRN_hi", "s"), ("klenN", "s"), ("m0N", "s"),
               ("n0N", "s"),
               ("cT_lo", "s"), ("cT_hi", "s"), ("crecT", "s"),
               ("stride_l", "s"), ("stride_r", "s"), ("cm2", "s"), ("alpha", "s"), ("sw_epi", "s")]
        ops += [(f"voffL{j}", "v") for j in range(self.nl)] + [(f"voffR{j}", "v") for j in range(self.nr)]
        if self.parity_bases:
            ops += [("amb0", "v"), ("amb1", "v"), ("bnb0", "v"), ("bnb1", "v")]
        else:
            ops += [(f"amb{i}", "v") for i in range(self.bm)] + [(f"bnb{j}", "v") for j in range(self.bn)]
        epi = (["ew_base", "ew_s", "rb_even", "rb_odd", "gb"] if out == "bf16"
               else ["fw_base", "fw_s", "frb", "fgb"])
        if mx:
            # the epilogue's per-lane bases are formed from the lane id inside the statement, in
            # operand registers free by then (the scale registers leave too few for them as inputs)
            self.lane_regs = {n: f"v{self.vop0 + 56 + k}" for k, n in enumerate(epi)}
            ops += [("scT_lo", "s"), ("scT_hi", "s"), ("scN_lo", "s"), ("scN_hi", "s"), ("stride_sc", "s"),
                    ("scrd", "s"), ("scw", "s"), ("vsc", "v"), ("vscb", "v")]
        else:
            self.lane_regs = {}
            ops += [(n, "v") for n in epi]
        self.operands = ops
        self.op = {name: f"%{i}" for i, (name, _) in enumerate(ops)}
        # MFMA order within a stage: m-block 0 across all n-blocks first, then the other m-blocks
        # column by column; m-block 0's registers free up after its row, an n-block's after its
        # column, so the next stage's operands are read spread over the stage.
        self.order = [(0, j) for j in range(self.bn)] + [(i, j) for j in range(self.bn) for i in range(1, self.bm)]
        pos = {ij: n for n, ij in enumerate(self.order)}
        self.barrier_after = self.bn - 1
        reads = {self.bn - 1: [("am", 0)]}
        for j in range(self.bn):
            reads.setdefault(pos[(self.bm - 1, j)], []).append(("bn", j))
        for i in range(1, self.bm):
            reads.setdefault(pos[(i, self.bn - 1)], []).append(("am", i))
        self.reads_after = reads
        free = [n for n in range(self.bn, len(self.order) - 1) if n not in reads]
        assert len(free) >= self.loads, self.name
        self.dma_after = free[:self.loads]
        self.setup_after = (0, 1, 2)
        assert self.vsc0 - 2 >= (20 if mx else 28) and self.vop0 % 2 == 0 and (out != "bf16" or self.e_stores + self.loads <= 63)
        assert self.nl * 4 * 1024 == KS * tm and self.nr * 4 * 1024 == KS * tn

    def acc(self, i, j):
        """Accumulator registers of block (m-block i, n-block j): blocks 0-15 in AGPRs, the rest in
        VGPRs from vacc0 up."""
        b = self.bn * i + j
        if b < 16:
            return "a", 16 * b
        return "v", self.vacc0 + 16 * (b - 16)

    def acc_range(self, i, j):
        kind, base = self.acc(i, j)
        return f"{kind}[{base}:{base + 15}]"

    def am(self, i):
        return self.vop0 + 8 * i

    def scale_reg(self, side, b):
        """(register, half) holding this lane's e8m0 scale of LHS m-block b (side "am") or RHS
        n-block b (side "bn"): bits 0-7 (half 0) or 16-23 (half 1)."""
        r, h = self.scale_map[(side, b)]
        return self.vsc0 + r, h

    def lane_value(self, name):
        """A per-lane epilogue base: an input operand, or (MX) the register the statement forms it in."""
        return self.lane_regs.get(name) or self.op[name]

    def bn_reg(self, j):
        return self.vop0 + 8 * self.bm + 8 * j

    def read_base(self, side, b):
        """(base operand, extra immediate) of block b's first transposed read."""
        if self.parity_bases:
            return self.op[f"{side}b{b & 1}"], 32 * b
        return self.op[f"{side}b{b}"], 0


CONFIGS = (Config(256, 384), Config(320, 320), Config(320, 320, "f32"), Config(320, 320, "f32acc"),
           Config(320, 320, mx=True))


class Gen:
    def __init__(self, cfg=CONFIGS[0]):
        self.cfg = cfg
        self.OP = cfg.op
        self.lines = []
        self.nlabel = 0
        self.nlds = 0           # LDS reads issued in the current read sequence (MX half-load waits)
        self.lo_at = {}

    def emit(self, s):
        self.lines.append(s)

    def label(self, stem):
        self.nlabel += 1
        return f".Lggw_{stem}{self.nlabel}_%="

    def capture(self, fn, *args):
        """The lines fn would emit, without emitting them."""
        saved, self.lines = self.lines, []
        fn(*args)
        out, self.lines = self.lines, saved
        return out

    # ---------------------------------------------------------------- vm model

    def wait_oldest(self):
        """Wait for the oldest issued, not yet awaited stage; pop it from the model. vmcnt is
        rounded down to one of the counts this kernel can produce (a stricter wait is safe)."""
        s, OP, c = SGPR, self.OP, self.cfg
        self.emit(f"s_sub_u32 {s['NEED']}, {OP['vmt']}, {OP['q0']}")
        self.emit(f"s_mov_b32 {OP['q0']}, {OP['q1']}")
        self.emit(f"s_mov_b32 {OP['q1']}, {OP['q2']}")
        self.emit(f"s_sub_u32 {OP['np']}, {OP['np']}, 1")
        counts = sorted({min(n, 63) for n in (c.e_stores + c.loads, c.e_stores, 2 * c.loads, c.loads)}, reverse=True)
        done = self.label("wdone")
        tgt = {n: self.label(f"w{n}_") for n in counts}
        self.emit(f"s_cmp_eq_u32 {s['NEED']}, {c.loads}")        # the steady state: one stage behind
        self.emit(f"s_cbranch_scc1 {tgt[c.loads]}")
        for n in counts:
            self.emit(f"s_cmp_ge_u32 {s['NEED']}, {n}")
            self.emit(f"s_cbranch_scc1 {tgt[n]}")
        self.emit("s_waitcnt vmcnt(0)")
        self.emit(f"s_branch {done}")
        for n in counts:
            self.emit(f"{tgt[n]}:")
            self.emit(f"s_waitcnt vmcnt({n})")
            self.emit(f"s_branch {done}")
        self.emit(f"{done}:")

    # ---------------------------------------------------------------- issue

    def issue_setup(self):
        """Buffer resources of the cursor's stage and this wave's LDS-DMA base in slot ISLOT."""
        s, OP, e = SGPR, self.OP, self.emit
        e(f"s_min_i32 {s['T']}, {s['REM']}, {KS}")
        e(f"s_max_i32 {s['T']}, {s['T']}, 0")
        e(f"s_mul_i32 {s['RL2']}, {s['T']}, {OP['stride_l']}")
        e(f"s_sub_u32 {s['RL2']}, {s['RL2']}, {s['CM0']}")
        e(f"s_mul_i32 {s['RR2']}, {s['T']}, {OP['stride_r']}")
        e(f"s_sub_u32 {s['RR2']}, {s['RR2']}, {s['CN0']}")
        e(f"s_mov_b32 {s['RL0']}, {s['BL0']}")
        e(f"s_and_b32 {s['RL1']}, {s['BL1']}, 0xffff")
        e(f"s_mov_b32 {s['RL3']}, 0x{WORD3:x}")
        e(f"s_mov_b32 {s['RR0']}, {s['BR0']}")
        e(f"s_and_b32 {s['RR1']}, {s['BR1']}, 0xffff")
        e(f"s_mov_b32 {s['RR3']}, 0x{WORD3:x}")
        e(f"s_add_u32 {s['IB']}, {OP['lds_base']}, {s['ISLOT']}")
        e(f"s_add_u32 {s['IB']}, {s['IB']}, {OP['w1k']}")
        if self.cfg.mx:
            # this wave's e8m0 row: blocks (valid tokens + 31) / 32 of the stage are in range,
            # each 320 bytes from the tile's column (the row stride is at least 320)
            e(f"s_add_u32 {s['T2']}, {s['T']}, 31")
            e(f"s_lshr_b32 {s['T2']}, {s['T2']}, 5")
            e(f"s_sub_u32 {s['T2']}, {s['T2']}, 1")
            e(f"s_mul_i32 {s['RS2']}, {s['T2']}, {OP['stride_sc']}")
            e(f"s_add_u32 {s['RS2']}, {s['RS2']}, 320")
            e(f"s_mov_b32 {s['RS0']}, {s['BS0']}")
            e(f"s_and_b32 {s['RS1']}, {s['BS1']}, 0xffff")
            e(f"s_mov_b32 {s['RS3']}, 0x{WORD3:x}")

    def issue_dma(self, j):
        """LDS-DMA instruction j of the stage (first the nl LHS rows, then the nr RHS rows)."""
        s, OP, e, c = SGPR, self.OP, self.emit, self.cfg
        if j < c.nl:
            e(f"s_add_u32 m0, {s['IB']}, {4096 * j}")
            e("s_nop 0")
            e(f"buffer_load_dwordx4 {OP[f'voffL{j}']}, {s['RL']}, 0 offen lds")
        elif j == c.nl + c.nr:
            # MX: lanes 0-39 carry the two 320-byte e8m0 rows of the wave's side (both waves of a side
            # write the same bytes); the other lanes' offsets are out of range (zeros into the rest
            # of the side's 1 KiB)
            e(f"s_lshr_b32 {s['T']}, {s['ISLOT']}, 4")
            e(f"s_add_u32 m0, {s['T']}, {OP['scw']}")
            e("s_nop 0")
            e(f"buffer_load_dwordx4 {OP['vsc']}, {s['RS']}, 0 offen lds")
        else:
            jj = j - c.nl
            e(f"s_add_u32 m0, {s['IB']}, {c.rhs_off + 4096 * jj}")
            e("s_nop 0")
            e(f"buffer_load_dwordx4 {OP[f'voffR{jj}']}, {s['RR']}, 0 offen lds")

    def issue_finish(self):
        """Model: loads more operations, the count right after this stage remembered; advance the
        cursor to its next stage and slot."""
        s, OP, e, c = SGPR, self.OP, self.emit, self.cfg
        e(f"s_add_u32 {OP['vmt']}, {OP['vmt']}, {c.loads}")
        for n, q in enumerate(("q0", "q1", "q2")):
            e(f"s_cmp_eq_u32 {OP['np']}, {n}")
            e(f"s_cselect_b32 {OP[q]}, {OP['vmt']}, {OP[q]}")
        e(f"s_add_u32 {OP['np']}, {OP['np']}, 1")
        e(f"s_add_u32 {s['IDX']}, {s['IDX']}, 1")
        e(f"s_sub_i32 {s['REM']}, {s['REM']}, {KS}")
        e(f"s_lshl_b32 {s['T']}, {OP['stride_l']}, 6")
        e(f"s_add_u32 {s['BL0']}, {s['BL0']}, {s['T']}")
        e(f"s_addc_u32 {s['BL1']}, {s['BL1']}, 0")
        e(f"s_lshl_b32 {s['T']}, {OP['stride_r']}, 6")
        e(f"s_add_u32 {s['BR0']}, {s['BR0']}, {s['T']}")
        e(f"s_addc_u32 {s['BR1']}, {s['BR1']}, 0")
        if c.mx:
            e(f"s_lshl_b32 {s['T']}, {OP['stride_sc']}, 1")
            e(f"s_add_u32 {s['BS0']}, {s['BS0']}, {s['T']}")
            e(f"s_addc_u32 {s['BS1']}, {s['BS1']}, 0")
        e(f"s_add_u32 {s['ISLOT']}, {s['ISLOT']}, {c.slot}")
        e(f"s_cmp_ge_u32 {s['ISLOT']}, {c.slot * SLOTS}")
        e(f"s_cselect_b32 {s['T']}, {c.slot * SLOTS}, 0")
        e(f"s_sub_u32 {s['ISLOT']}, {s['ISLOT']}, {s['T']}")

    def issue_core(self):
        """Issue the cursor's stage into slot ISLOT and advance the cursor."""
        self.issue_setup()
        for j in range(self.cfg.loads):
            self.issue_dma(j)
        self.issue_finish()

    def cursor_prep(self):
        """Before a stage that may issue: move the cursor to the next tile once this one is fully
        issued (the next tile's first two stages are the cursor's limit there); SCC = the cursor
        has a stage to issue."""
        s, OP, e = SGPR, self.OP, self.emit
        nosw = self.label("nosw")
        e(f"s_cmp_eq_u32 {s['INT']}, 1")
        e(f"s_cbranch_scc0 {nosw}")
        e(f"s_cmp_eq_u32 {s['IDX']}, {s['S']}")
        e(f"s_cbranch_scc0 {nosw}")
        e(f"s_mov_b32 {s['INT']}, 0")
        e(f"s_mov_b32 {s['IDX']}, 0")
        e(f"s_mov_b32 {s['REM']}, {OP['klenN']}")
        e(f"s_add_u32 {s['T']}, {OP['klenN']}, {KS - 1}")
        e(f"s_lshr_b32 {s['T']}, {s['T']}, 6")
        e(f"s_min_u32 {s['LIM']}, {s['T']}, 2")
        e(f"s_mov_b32 {s['BL0']}, {OP['bLN_lo']}")
        e(f"s_mov_b32 {s['BL1']}, {OP['bLN_hi']}")
        e(f"s_mov_b32 {s['BR0']}, {OP['bRN_lo']}")
        e(f"s_mov_b32 {s['BR1']}, {OP['bRN_hi']}")
        e(f"s_mov_b32 {s['CM0']}, {OP['m0N']}")
        e(f"s_mov_b32 {s['CN0']}, {OP['n0N']}")
        if self.cfg.mx:
            e(f"s_mov_b32 {s['BS0']}, {OP['scN_lo']}")
            e(f"s_mov_b32 {s['BS1']}, {OP['scN_hi']}")
        e(f"{nosw}:")
        e(f"s_cmp_lt_u32 {s['IDX']}, {s['LIM']}")

    # ---------------------------------------------------------------- operands

    def read_block(self, side, b, slot):
        c, e = self.cfg, self.emit
        base, extra = c.read_base(side, b)
        pitch = c.tm if side == "am" else c.tn
        reg0 = c.am(b) if side == "am" else c.bn_reg(b)
        e(f"v_add_u32 {c.vt}, {slot}, {base}")
        for n, dt in enumerate(TOK_OFFS):
            r = reg0 + 2 * n
            e(f"ds_read_b64_tr_b8 v[{r}:{r + 1}], {c.vt} offset:{extra + dt * pitch}")
        self.nlds += len(TOK_OFFS)
        if c.mx:
            # the lane's e8m0 scale of block b (row l % 32, token block l / 32 of the stage)
            reg, half = c.scale_reg(side, b)
            sslot = SGPR["NSS"] if side == "am" else SGPR["NSSR"]
            e(f"v_add_u32 {c.vt}, {sslot}, {self.OP['vscb']}")
            if half:
                # the load of the register's other half has completed (at most `after` LDS reads
                # issued since it may still be in flight)
                after = self.nlds - self.lo_at[reg] - 1
                e(f"s_waitcnt lgkmcnt({min(after, 15)})")
            else:
                self.lo_at[reg] = self.nlds
            e(f"ds_read_u8{'_d16_hi' if half else ''} v{reg}, {c.vt} offset:{32 * b}")
            self.nlds += 1

    def scale_slot(self, slot):
        """NSS / NSSR = the scale slot offsets (LHS / RHS rows) that go with stage slot `slot`."""
        s = SGPR
        self.emit(f"s_lshr_b32 {s['NSS']}, {slot}, 4")
        self.emit(f"s_add_u32 {s['NSSR']}, {s['NSS']}, {self.OP['scrd']}")

    def mfma(self, i, j, first):
        c = self.cfg
        d = c.acc_range(i, j)
        src = "0" if first else d
        a, b = c.bn_reg(j), c.am(i)
        if c.mx:
            # scale of A (RHS n-block j) and of B (LHS m-block i): the byte op_sel_hi picks (0 or 2)
            ra, ha = c.scale_reg("bn", j)
            rb, hb = c.scale_reg("am", i)
            self.emit(f"v_mfma_scale_f32_32x32x64_f8f6f4 {d}, v[{a}:{a + 7}], v[{b}:{b + 7}], {src}, v{ra}, v{rb} "
                      f"op_sel_hi:[{ha},{hb},0] cbsz:1")
            return
        self.emit(f"v_mfma_f32_32x32x64_f8f6f4 {d}, v[{a}:{a + 7}], v[{b}:{b + 7}], {src} cbsz:1")

    # ---------------------------------------------------------------- one stage

    def stage(self, first, last, issue):
        """Stage k: its operands are in registers (read during stage k-1, or at tile entry for the
        first stage); CS = its slot. After the first row of MFMAs every read of slot CS has
        completed; unless last, the wave then waits for stage k+1's loads and passes the barrier
        (stage k+1 published, slot CS free); stage k+1's operands are read as their registers free
        up, and with issue the cursor's next stage goes into slot CS one LDS-DMA instruction per
        MFMA gap."""
        s, e, c = SGPR, self.emit, self.cfg
        if not last:
            e(f"s_add_u32 {s['NS']}, {s['CS']}, {c.slot}")
            e(f"s_cmp_ge_u32 {s['NS']}, {c.slot * SLOTS}")
            e(f"s_cselect_b32 {s['T']}, {c.slot * SLOTS}, 0")
            e(f"s_sub_u32 {s['NS']}, {s['NS']}, {s['T']}")
            if c.mx:
                self.scale_slot(s["NS"])
        setup = self.capture(self.issue_setup) if issue else []
        third = (len(setup) + 2) // 3
        pieces = [setup[:third], setup[third:2 * third], setup[2 * third:]]
        # the previous stage's reads ended with the last n-block and the last m-block (rb reads
        # each); lgkmcnt(15) leaves at most 15 of them in flight: m-block 0 and the n-blocks before
        # the last are in
        e("s_waitcnt lgkmcnt(0)" if first else "s_waitcnt lgkmcnt(15)")
        self.nlds, self.lo_at = 0, {}
        for n, (i, j) in enumerate(c.order):
            if not first and n == c.bn - 1:
                e(f"s_waitcnt lgkmcnt({c.rb})")
            self.mfma(i, j, first)
            if issue and n in c.setup_after:
                for line in pieces[c.setup_after.index(n)]:
                    e(line)
            if n == c.barrier_after:
                e("s_waitcnt lgkmcnt(0)")
                if not last:
                    self.wait_oldest()
                    e("s_barrier")
            if last:
                continue
            for side, b in c.reads_after.get(n, []):
                self.read_block(side, b, s["NS"])
            if issue and n in c.dma_after:
                k = c.dma_after.index(n)
                self.issue_dma(k)
                if k == c.loads - 1:
                    self.issue_finish()

    def variant_pair(self, first):
        """A stage that is not the tile's last: with or without a stage to issue."""
        e = self.emit
        noiss, join = self.label("noiss"), self.label("join")
        self.cursor_prep()
        e(f"s_cbranch_scc0 {noiss}")
        self.stage(first=first, last=False, issue=True)
        e(f"s_branch {join}")
        e(f"{noiss}:")
        self.stage(first=first, last=False, issue=False)
        e(f"{join}:")

    # ---------------------------------------------------------------- epilogue

    def c_resource(self):
        s, OP, e = SGPR, self.OP, self.emit
        e(f"s_mov_b32 {s['RC0']}, {OP['cT_lo']}")
        e(f"s_and_b32 {s['RC1']}, {OP['cT_hi']}, 0xffff")
        e(f"s_mov_b32 {s['RC2']}, {OP['crecT']}")
        e(f"s_mov_b32 {s['RC3']}, 0x{WORD3:x}")

    def store_offset(self, i, row, j0, lane_base):
        """vt2 = byte offset of this wave's tile row 32 i + row (lane part in lane_base), columns
        from block j0 (32 j0) on."""
        s, OP, e, c = SGPR, self.OP, self.emit, self.cfg
        e(f"s_mul_i32 {s['T']}, {OP['cm2']}, {32 * i + row}")
        e(f"s_add_u32 {s['T']}, {s['T']}, {OP['sw_epi']}")
        if j0 > 0:
            e(f"s_add_u32 {s['T']}, {s['T']}, {64 * j0}")
        elif j0 < 0:
            e(f"s_sub_u32 {s['T']}, {s['T']}, {-64 * j0}")
        e(f"v_add_u32 {c.vt2}, {s['T']}, {c.lane_value(lane_base)}")

    def by_half(self, body):
        """body(wn) for this wave's half of the tile's columns: the right-half waves (wn = bit 11
        of w1k) run their own code where the two halves' passes differ (an odd block count)."""
        c, e = self.cfg, self.emit
        if not c.joint:
            body(0)
            return
        right, done = self.label("wn1_"), self.label("wndone")
        e(f"s_bitcmp1_b32 {self.OP['w1k']}, 11")
        e(f"s_cbranch_scc1 {right}")
        body(0)
        e(f"s_branch {done}")
        e(f"{right}:")
        body(1)
        e(f"{done}:")

    # stores of a two-block pass: (row offset, read base index, read immediate); read-back k gives
    # lane l row 8 k + l / 8, chunk l % 8 (rows 16.. at +2048 of the rows-0.. bases)
    PAIR_STORES = [(8 * k, k % 2, 2048 if k >= 2 else 0) for k in range(4)]

    @staticmethod
    def joint_stores(wn):
        """The joint pass's stores of wave half wn: rows 0-15 (left) or 16-31 (right) of the shared
        line, as (row offset, read base index, read immediate)."""
        return Gen.PAIR_STORES[2 * wn:2 * wn + 2]

    def joint_col(self, wn):
        """First block of the shared line in this wave's column frame (the right half's is -1)."""
        return self.cfg.bn - 1 if wn == 0 else -1

    def epilogue(self):
        if self.cfg.out != "bf16":
            return self.epilogue_f32()
        s, OP, e, c = SGPR, self.OP, self.emit, self.cfg
        v0 = c.vop0                      # the operand registers are free here
        tacc, tmul, tcvt = v0, v0 + 4, v0 + 8
        waddr, rbase, dset = v0 + 10, v0 + 18, (v0 + 24, v0 + 40)
        e("s_nop 7")
        e("s_nop 7")
        e("s_nop 7")
        e("s_barrier")   # every wave is past its reads of the last stage's slot
        self.lane_values()
        e(f"s_add_u32 {s['EPI']}, {OP['lds_base']}, {s['CS']}")
        e(f"s_lshl_b32 {s['T']}, {OP['w1k']}, 2")
        e(f"s_add_u32 {s['EPI']}, {s['EPI']}, {s['T']}")
        # staging write address of chunk cc: row l % 32, chunk cc ^ swz(row), half l / 32
        for cc in range(8):
            e(f"v_xor_b32 v{tcvt}, {cc}, {c.lane_value('ew_s')}")
            e(f"v_lshlrev_b32 v{tcvt}, 4, v{tcvt}")
            e(f"v_add3_u32 v{waddr + cc}, v{tcvt}, {c.lane_value('ew_base')}, {s['EPI']}")
        e(f"v_add_u32 v{rbase}, {s['EPI']}, {c.lane_value('rb_even')}")
        e(f"v_add_u32 v{rbase + 1}, {s['EPI']}, {c.lane_value('rb_odd')}")
        self.c_resource()
        xw, xr = c.epi_x, c.epi_x + 4    # joint pass: write and read addresses in the shared region
        if c.joint:
            # IB (free in the epilogue) = the shared region of this wave row: slot + 16 KiB +
            # wm * 8 KiB, two 4 KiB buffers by m-block parity; T2 = its distance from EPI
            e(f"s_and_b32 {s['T']}, {OP['w1k']}, 1024")
            e(f"s_lshl_b32 {s['T']}, {s['T']}, 3")
            e(f"s_add_u32 {s['IB']}, {OP['lds_base']}, {s['CS']}")
            e(f"s_add_u32 {s['IB']}, {s['IB']}, {s['T']}")
            e(f"s_add_u32 {s['IB']}, {s['IB']}, 16384")
            e(f"s_sub_u32 {s['T2']}, {s['IB']}, {s['EPI']}")
            e(f"v_add_u32 v{xr}, {s['IB']}, {c.lane_value('rb_even')}")
            e(f"v_add_u32 v{xr + 1}, {s['IB']}, {c.lane_value('rb_odd')}")

        def block_to_lds(i, j, addr, off=0):
            """Scale, round to bf16 and write block (i, j): lane (r, h) writes half h of chunks
            addr[0..3] of row r."""
            kind, base = c.acc(i, j)
            for g in range(4):
                src = []
                for r in range(4):
                    reg = base + 4 * g + r
                    if kind == "a":
                        e(f"v_accvgpr_read_b32 v{tacc + r}, a{reg}")
                        src.append(f"v{tacc + r}")
                    else:
                        src.append(f"v{reg}")
                for r in range(4):
                    e(f"v_mul_f32 v{tmul + r}, {OP['alpha']}, {src[r]}")
                e(f"v_cvt_pk_bf16_f32 v{tcvt}, v{tmul}, v{tmul + 1}")
                e(f"v_cvt_pk_bf16_f32 v{tcvt + 1}, v{tmul + 2}, v{tmul + 3}")
                e(f"ds_write_b64 v{addr[g]}, v[{tcvt}:{tcvt + 1}]" + (f" offset:{off}" if off else ""))

        def passes(wn):
            pairs = c.pairs_wn1 if wn else c.pairs
            if c.joint:
                # this half's chunks of the shared line: 0-3 (left) or 4-7 (right) of each row
                for g in range(4):
                    e(f"v_add_u32 v{xw + g}, {s['T2']}, v{waddr + 4 * wn + g}")
            npass = 0
            for i in range(c.bm):
                if c.joint:
                    off = 4096 * (i % 2)
                    block_to_lds(i, c.joint_block[wn], [xw + g for g in range(4)], off)
                    e("s_waitcnt lgkmcnt(0)")
                    e("s_barrier")   # both halves' blocks of the shared line are in LDS
                    dbase = dset[npass % 2]
                    npass += 1
                    stores = self.joint_stores(wn)
                    for k, (_, rb, imm) in enumerate(stores):
                        d = dbase + 4 * k
                        e(f"ds_read_b128 v[{d}:{d + 3}], v{xr + rb} offset:{off + imm}")
                    e("s_waitcnt lgkmcnt(0)")
                    for k, (row, _, _) in enumerate(stores):
                        d = dbase + 4 * k
                        self.store_offset(i, row, self.joint_col(wn), "gb")
                        e(f"buffer_store_dwordx4 v[{d}:{d + 3}], {c.vt2}, {s['RC']}, 0 offen nt")
                for blocks in pairs:
                    dbase = dset[npass % 2]
                    npass += 1
                    for jj, j in enumerate(blocks):
                        block_to_lds(i, j, [waddr + 4 * jj + g for g in range(4)])
                    for k, (_, rb, imm) in enumerate(self.PAIR_STORES):
                        d = dbase + 4 * k
                        e(f"ds_read_b128 v[{d}:{d + 3}], v{rbase + rb} offset:{imm}")
                    e("s_waitcnt lgkmcnt(0)")
                    for k, (row, _, _) in enumerate(self.PAIR_STORES):
                        d = dbase + 4 * k
                        self.store_offset(i, row, blocks[0], "gb")
                        e(f"buffer_store_dwordx4 v[{d}:{d + 3}], {c.vt2}, {s['RC']}, 0 offen nt")
        self.by_half(passes)
        e(f"s_add_u32 {OP['vmt']}, {OP['vmt']}, {c.e_stores}")

    def lane_values(self):
        """MX: form the bf16 epilogue's per-lane bases from the lane id (the other configurations
        take them as operands), restating vark_wide.h's set-up: staging writes at row rl = l % 32,
        half hl = l / 32 (ew_base = 128 rl + 8 hl, ew_s = (rl / 2) % 8); read-back rows rr = l / 8,
        chunk rc = l % 8 (rb_even = 128 rr + 16 (rc ^ rs), rb_odd = 128 (8 + rr) + 16 (rc ^ rs ^ 4),
        rs = rr / 2; gb = rr * cm2 + 16 rc)."""
        c, e, OP = self.cfg, self.emit, self.OP
        if not c.lane_regs:
            return
        R = c.lane_regs
        t = c.vop0 + 56 + len(R)
        ln, t0, t1, t2, rr, rc = (f"v{t + k}" for k in range(6))
        assert t + 6 <= c.vacc0
        e(f"v_mbcnt_lo_u32_b32 {ln}, -1, 0")
        e(f"v_mbcnt_hi_u32_b32 {ln}, -1, {ln}")
        e(f"v_and_b32 {t0}, 31, {ln}")
        e(f"v_lshrrev_b32 {t1}, 5, {ln}")
        e(f"v_lshlrev_b32 {t0}, 7, {t0}")
        e(f"v_lshl_add_u32 {R['ew_base']}, {t1}, 3, {t0}")
        e(f"v_bfe_u32 {R['ew_s']}, {ln}, 1, 3")
        e(f"v_lshrrev_b32 {rr}, 3, {ln}")
        e(f"v_and_b32 {rc}, 7, {ln}")
        e(f"v_lshrrev_b32 {t0}, 4, {ln}")
        e(f"v_xor_b32 {t1}, {rc}, {t0}")
        e(f"v_lshlrev_b32 {t1}, 4, {t1}")
        e(f"v_lshl_add_u32 {R['rb_even']}, {rr}, 7, {t1}")
        e(f"v_xor_b32 {t1}, 4, {t0}")
        e(f"v_xor_b32 {t1}, {t1}, {rc}")
        e(f"v_lshlrev_b32 {t1}, 4, {t1}")
        e(f"v_add_u32 {t2}, 8, {rr}")
        e(f"v_lshl_add_u32 {R['rb_odd']}, {t2}, 7, {t1}")
        e(f"v_mul_lo_u32 {t2}, {rr}, {OP['cm2']}")
        e(f"v_lshl_add_u32 {R['gb']}, {rc}, 4, {t2}")

    def f32_store_offset(self, i, j, k):
        """vt2 = byte offset of this wave's tile rows 32 i + 8 k + l / 8, columns 32 j + 4 (l % 8)
        (fp32)."""
        s, OP, e, c = SGPR, self.OP, self.emit, self.cfg
        e(f"s_mul_i32 {s['T']}, {OP['cm2']}, {2 * (32 * i + 8 * k)}")
        e(f"s_add_u32 {s['T']}, {s['T']}, {OP['sw_epi']}")
        if j:
            e(f"s_add_u32 {s['T']}, {s['T']}, {128 * j}")
        e(f"v_add_u32 {c.vt2}, {s['T']}, {OP['fgb']}")

    def epilogue_f32(self):
        """fp32 C, one 32 x 32 block per pass through a private 4 KiB LDS region: lane (r = l % 32,
        h = l / 32) writes its four 16-byte row pieces (chunk 2 g + h of row r, chunk c stored at
        c ^ (((r >> 1) & 3) << 1)); read-back k (0..3) gives lane l row 8 k + l / 8, chunk l % 8, so
        each 1 KiB store covers 8 whole 128-byte row segments. Accumulating, the product, rounded to
        fp32 first, is added to the old values, whose loads run ahead of the pass that adds them:
        the passes take the blocks held in VGPRs first, and each such block's 16 registers, free once
        its pass has scaled them, join the three spare 16-register buffers that the old values load
        into, so later passes keep up to 12 passes of loads in flight (counted vmcnt)."""
        s, OP, e, c = SGPR, self.OP, self.emit, self.cfg
        acc_mode = c.out == "f32acc"
        v0 = c.vop0                      # the operand registers are free here
        tacc, tmul, waddr, rbase = v0, v0 + 4, v0 + 8, v0 + 12
        dset = v0 + 16                   # the pass's staged results (a store reads its data at issue)
        look = 2                         # passes of old-value loads in flight ahead of the current
        oset = [v0 + 32 + 16 * k for k in range(look + 1)]
        assert oset[-1] + 16 <= c.vacc0
        e("s_nop 7")
        e("s_nop 7")
        e("s_nop 7")
        e("s_barrier")   # every wave is past its reads of the last stage's slot
        e(f"s_add_u32 {s['EPI']}, {OP['lds_base']}, {s['CS']}")
        e(f"s_lshl_b32 {s['T']}, {OP['w1k']}, 2")
        e(f"s_add_u32 {s['EPI']}, {s['EPI']}, {s['T']}")
        for g in range(4):
            e(f"v_xor_b32 v{tacc}, {g}, {OP['fw_s']}")
            e(f"v_lshlrev_b32 v{tacc}, 5, v{tacc}")
            e(f"v_add3_u32 v{waddr + g}, v{tacc}, {OP['fw_base']}, {s['EPI']}")
        e(f"v_add_u32 v{rbase}, {s['EPI']}, {OP['frb']}")
        self.c_resource()
        blocks = [(i, j) for i in range(c.bm) for j in range(c.bn)]
        if acc_mode:
            # blocks held in VGPRs first: their registers become old-value buffers after their pass
            blocks.sort(key=lambda ij: c.acc(*ij)[0] != "v")
        P = len(blocks)
        pool = list(oset)        # free 16-register buffers for old values
        buf = {}                 # pass -> its old-value buffer
        vm_log = []              # vector memory operations of this epilogue, in issue order
        issued = [0]             # passes whose old-value loads are out

        def load_old(n, o0):
            i, j = blocks[n]
            for k in range(4):
                o = o0 + 4 * k
                self.f32_store_offset(i, j, k)
                e(f"buffer_load_dwordx4 v[{o}:{o + 3}], {c.vt2}, {s['RC']}, 0 offen nt")
                vm_log.append(("L", n))

        def issue_loads():
            while issued[0] < P and pool:
                n = issued[0]
                buf[n] = pool.pop(0)
                load_old(n, buf[n])
                issued[0] += 1

        if acc_mode:
            pool = pool[:look]   # two passes ahead at first, as many as buffers free up later
            issue_loads()
            pool = list(oset[look:])
        for n, (i, j) in enumerate(blocks):
            kind, base = c.acc(i, j)
            for g in range(4):
                src = []
                for r in range(4):
                    reg = base + 4 * g + r
                    if kind == "a":
                        e(f"v_accvgpr_read_b32 v{tacc + r}, a{reg}")
                        src.append(f"v{tacc + r}")
                    else:
                        src.append(f"v{reg}")
                for r in range(4):
                    e(f"v_mul_f32 v{tmul + r}, {OP['alpha']}, {src[r]}")
                e(f"ds_write_b128 v{waddr + g}, v[{tmul}:{tmul + 3}]")
            for k in range(4):
                e(f"ds_read_b128 v[{dset + 4 * k}:{dset + 4 * k + 3}], v{rbase} offset:{1024 * k}")
            if acc_mode:
                if kind == "v":
                    pool.append(base)          # scaled above: the block's registers are free
                issue_loads()
                # issued after this pass's old values: later passes' loads and the stores of the
                # passes since (vector memory counts complete in issue order; vmcnt holds 63)
                last = max(k for k, op in enumerate(vm_log) if op == ("L", n))
                e(f"s_waitcnt vmcnt({min(len(vm_log) - 1 - last, 63)})")
            e("s_waitcnt lgkmcnt(0)")
            if acc_mode:
                o0 = buf[n]
                for r in range(16):
                    e(f"v_add_f32 v{dset + r}, v{dset + r}, v{o0 + r}")
            for k in range(4):
                self.f32_store_offset(i, j, k)
                e(f"buffer_store_dwordx4 v[{dset + 4 * k}:{dset + 4 * k + 3}], {c.vt2}, {s['RC']}, 0 offen nt")
                vm_log.append(("S", n))
            if acc_mode:
                pool.append(buf[n])            # added: the buffer takes a later pass's loads
        e(f"s_add_u32 {OP['vmt']}, {OP['vmt']}, {c.e_stores}")

    def zero_epilogue(self):
        """A tile without tokens: zeros straight from registers, the same stores per wave (fp32
        accumulation: C += 0, nothing to do)."""
        e, c = self.emit, self.cfg
        if c.out == "f32acc":
            e(f"s_add_u32 {self.OP['vmt']}, {self.OP['vmt']}, 0")
            return
        if c.out == "f32":
            z = c.vop0 + 16
            for r in range(z, z + 4):
                e(f"v_mov_b32 v{r}, 0")
            self.c_resource()
            for i in range(c.bm):
                for j in range(c.bn):
                    for k in range(4):
                        self.f32_store_offset(i, j, k)
                        e(f"buffer_store_dwordx4 v[{z}:{z + 3}], {c.vt2}, {SGPR['RC']}, 0 offen nt")
            e(f"s_add_u32 {self.OP['vmt']}, {self.OP['vmt']}, {c.e_stores}")
            return
        z = c.vop0 + 24
        for r in range(z, z + 4):
            e(f"v_mov_b32 v{r}, 0")
        self.lane_values()
        self.c_resource()

        def zeros(wn):
            for i in range(c.bm):
                if c.joint:
                    for row, _, _ in self.joint_stores(wn):
                        self.store_offset(i, row, self.joint_col(wn), "gb")
                        e(f"buffer_store_dwordx4 v[{z}:{z + 3}], {c.vt2}, {SGPR['RC']}, 0 offen nt")
                for blocks in (c.pairs_wn1 if wn else c.pairs):
                    for row, _, _ in self.PAIR_STORES:
                        self.store_offset(i, row, blocks[0], "gb")
                        e(f"buffer_store_dwordx4 v[{z}:{z + 3}], {c.vt2}, {SGPR['RC']}, 0 offen nt")
        self.by_half(zeros)
        e(f"s_add_u32 {self.OP['vmt']}, {self.OP['vmt']}, {c.e_stores}")

    # ---------------------------------------------------------------- whole tile

    def tile(self):
        s, OP, e, c = SGPR, self.OP, self.emit, self.cfg
        e("s_nop 4")   # inputs may come from v_readfirstlane (VALU-written SGPRs) just before
        e(f"s_add_u32 {s['S']}, {OP['klenT']}, {KS - 1}")
        e(f"s_lshr_b32 {s['S']}, {s['S']}, 6")
        e(f"s_mul_i32 {s['CS']}, {OP['c0']}, {c.slot}")
        e(f"s_add_u32 {s['T']}, {OP['c0']}, {OP['nis']}")
        e(f"s_cmp_ge_u32 {s['T']}, {SLOTS}")
        e(f"s_cselect_b32 {s['T2']}, {SLOTS}, 0")
        e(f"s_sub_u32 {s['T']}, {s['T']}, {s['T2']}")
        e(f"s_mul_i32 {s['ISLOT']}, {s['T']}, {c.slot}")
        # cursor: this tile, at its first stage not yet issued
        e(f"s_mov_b32 {s['INT']}, 1")
        e(f"s_mov_b32 {s['IDX']}, {OP['nis']}")
        e(f"s_mov_b32 {s['LIM']}, {s['S']}")
        e(f"s_lshl_b32 {s['T']}, {OP['nis']}, 6")
        e(f"s_sub_i32 {s['REM']}, {OP['klenT']}, {s['T']}")
        e(f"s_lshl_b32 {s['T']}, {OP['stride_l']}, 6")
        e(f"s_mul_i32 {s['T']}, {s['T']}, {OP['nis']}")
        e(f"s_add_u32 {s['BL0']}, {OP['bLT_lo']}, {s['T']}")
        e(f"s_addc_u32 {s['BL1']}, {OP['bLT_hi']}, 0")
        e(f"s_lshl_b32 {s['T']}, {OP['stride_r']}, 6")
        e(f"s_mul_i32 {s['T']}, {s['T']}, {OP['nis']}")
        e(f"s_add_u32 {s['BR0']}, {OP['bRT_lo']}, {s['T']}")
        e(f"s_addc_u32 {s['BR1']}, {OP['bRT_hi']}, 0")
        e(f"s_mov_b32 {s['CM0']}, {OP['m0T']}")
        e(f"s_mov_b32 {s['CN0']}, {OP['n0T']}")
        if c.mx:
            e(f"s_lshl_b32 {s['T']}, {OP['stride_sc']}, 1")
            e(f"s_mul_i32 {s['T']}, {s['T']}, {OP['nis']}")
            e(f"s_add_u32 {s['BS0']}, {OP['scT_lo']}, {s['T']}")
            e(f"s_addc_u32 {s['BS1']}, {OP['scT_hi']}, 0")
        e("s_barrier")   # the previous tile's epilogue is done with its staging slot
        # top up to three stages of this tile in flight
        e(f"s_min_u32 {s['LIMTOP']}, {s['S']}, {SLOTS}")
        top, topdone = self.label("top"), self.label("topdone")
        e(f"{top}:")
        e(f"s_cmp_lt_u32 {s['IDX']}, {s['LIMTOP']}")
        e(f"s_cbranch_scc0 {topdone}")
        self.issue_core()
        e(f"s_branch {top}")
        e(f"{topdone}:")
        zero, end = self.label("zero"), self.label("end")
        e(f"s_cmp_eq_u32 {s['S']}, 0")
        e(f"s_cbranch_scc1 {zero}")
        self.wait_oldest()
        e("s_barrier")
        if c.mx:
            self.scale_slot(s["CS"])
        self.nlds, self.lo_at = 0, {}
        for i in range(c.bm):
            self.read_block("am", i, s["CS"])
        for j in range(c.bn):
            self.read_block("bn", j, s["CS"])
        first_last, loop, steady_last, epi = (self.label(x) for x in ("fl", "loop", "sl", "epi"))
        e(f"s_cmp_eq_u32 {s['S']}, 1")
        e(f"s_cbranch_scc1 {first_last}")
        self.variant_pair(first=True)
        e(f"s_mov_b32 {s['CS']}, {s['NS']}")
        e(f"s_mov_b32 {s['K']}, 1")
        e(f"{loop}:")
        e(f"s_add_u32 {s['T']}, {s['K']}, 1")
        e(f"s_cmp_eq_u32 {s['T']}, {s['S']}")
        e(f"s_cbranch_scc1 {steady_last}")
        self.variant_pair(first=False)
        e(f"s_mov_b32 {s['CS']}, {s['NS']}")
        e(f"s_add_u32 {s['K']}, {s['K']}, 1")
        e(f"s_branch {loop}")
        e(f"{first_last}:")
        self.stage(first=True, last=True, issue=False)
        e(f"s_branch {epi}")
        e(f"{steady_last}:")
        self.stage(first=False, last=True, issue=False)
        e(f"{epi}:")
        self.epilogue()
        e(f"s_branch {end}")
        e(f"{zero}:")
        self.zero_epilogue()
        e(f"{end}:")
        # the next tile's stages this cursor issued
        e(f"s_cmp_eq_u32 {s['INT']}, 0")
        e(f"s_cselect_b32 {OP['nis']}, {s['IDX']}, 0")


# ==================================================================== K-major (persistent fwd / dgrad)
#
# The persistent grouped GEMM C[r, :] = s_a s_b A[r, :] B[g]^T (persistent_wide.h) on the same
# one-wave-per-SIMD tile: 256 rows of A (C rows, the "am" side) x 320 rows of B (C columns, "bn"),
# both K-contiguous. The K axis goes in stages of 128 bytes, so every LDS-DMA row segment is one
# whole 128-byte line when the row stride is line-aligned (a 64-byte stage would ask the L2 for a
# line twice); a stage (256 + 320 rows x 128 bytes, 72 KiB) leaves room for two slots and the
# schedule tables. Per stage and wave two K-halves of 4 x 5 v_mfma_f32_32x32x64_f8f6f4; a half's
# operands (two ds_read_b128 per 32-row block) are read during the previous half as registers free
# up. The slot's next stage is requested from the barrier in the stage's second half on (18 LDS-DMA
# instructions per wave, 8 rows x 128 bytes each, one or two in every MFMA gap from the barrier's to
# the half's last), so a stage's loads have about one stage time to land. Spread over all 16 gaps
# rather than two or three in each of the 8 gaps without operand reads, they measured 2.4-3 %
# faster at the fwd sites: the 72 KiB the four waves request per stage take ~1150 cycles of the
# CU's texture-address unit, and a wave whose next load finds its queue full stops issuing MFMAs.
# K % 128 == 64 (K = 2880) makes the tile's last stage a half stage: its second half is neither
# computed nor read.
KSLOTS = 2
KKS = 128                    # K bytes per stage


class KConfig(Config):
    def __init__(self, tm, tn, a_e5m2):
        self.tm, self.tn = tm, tn
        self.a_e5m2 = a_e5m2
        self.out, self.mx, self.kmajor = "bf16", False, True
        self.name = f"pk{tm}x{tn}_" + ("e5m2" if a_e5m2 else "e4m3")
        self.bm, self.bn = tm // 64, tn // 64
        self.rhs_off = KKS * tm
        self.slot = KKS * (tm + tn)
        self.nl = KKS * tm // 4096
        self.nr = KKS * tn // 4096
        self.loads = self.nl + self.nr
        nblk = self.bm * self.bn
        assert 16 < nblk <= 32
        self.vacc0 = 256 - 16 * (nblk - 16)
        self.scale_map, self.nsl, self.nsr = {}, 0, 0
        self.vop0 = self.vacc0 - 8 * (self.bm + self.bn)
        self.vsc0 = self.vop0
        self.vt = f"v{self.vop0 - 2}"
        self.vt2 = f"v{self.vop0 - 1}"
        # the epilogue's joint-pass addresses below the operands: the 72 operand registers leave
        # no room above them before the VGPR accumulators
        self.epi_x = self.vop0 - 8
        self.vgpr_clobber = list(range(self.epi_x, 256))
        self.sgpr_clobber = list(range(56, 90))
        self.rb = 2                                     # two 128-bit reads per 32-row block
        self.joint = self.bn % 2 == 1
        self.pairs = [(2 * q, 2 * q + 1) for q in range(self.bn // 2)]
        self.pairs_wn1 = [(2 * q + 1, 2 * q + 2) for q in range(self.bn // 2)] if self.joint else self.pairs
        self.joint_block = (self.bn - 1, 0)
        self.e_stores = self.bm * (4 * len(self.pairs) + (2 if self.joint else 0))
        self.parity_bases = False
        ops = [("c0", "+s"), ("nis", "+s"), ("vmt", "+s"), ("q0", "+s"), ("q1", "+s"), ("q2", "+s"), ("np", "+s"),
               ("lds_base", "s"), ("w1k", "s"),
               ("bLT_lo", "s"), ("bLT_hi", "s"), ("bRT_lo", "s"), ("bRT_hi", "s"), ("klenT", "s"), ("recAT", "s"),
               ("recBT", "s"),
               ("bLN_lo", "s"), ("bLN_hi", "s"), ("bRN_lo", "s"), ("bRN_hi", "s"), ("klenN", "s"), ("recAN", "s"),
               ("recBN", "s"),
               ("cT_lo", "s"), ("cT_hi", "s"), ("crecT", "s"), ("cm2", "s"), ("alpha", "s"), ("sw_epi", "s")]
        ops += [(f"voffL{j}", "v") for j in range(self.nl)] + [(f"voffR{j}", "v") for j in range(self.nr)]
        ops += [(f"{side}{hl}{kh}", "v") for side in ("am", "bn") for kh in (0, 1) for hl in ("lo", "hi")]
        ops += [(n, "v") for n in ("ew_base", "ew_s", "rb_even", "rb_odd", "gb")]
        self.lane_regs = {}
        self.operands = ops
        self.op = {name: f"%{i}" for i, (name, _) in enumerate(ops)}
        self.order = [(0, j) for j in range(self.bn)] + [(i, j) for j in range(self.bn) for i in range(1, self.bm)]
        pos = {ij: n for n, ij in enumerate(self.order)}
        # the barrier that publishes the next stage and frees this one's slot: after MFMA 2 of the
        # second half, once the issue set-up (emitted after MFMAs 0-2) is complete; two MFMAs before the
        # end of the first row (where the wgrad kernels put it) measured 1.1-2.0 % faster at the fwd
        # sites, the stage's loads starting two gaps earlier; one or none before it would issue loads
        # from a half-built buffer resource
        self.barrier_after = 2
        reads = {self.bn - 1: [("am", 0)]}
        for j in range(self.bn):
            reads.setdefault(pos[(self.bm - 1, j)], []).append(("bn", j))
        for i in range(1, self.bm):
            reads.setdefault(pos[(i, self.bn - 1)], []).append(("am", i))
        self.reads_after = reads
        # a half's operand reads in issue order; at the next half's start every block up to the
        # n-block its (0, bn - 2) MFMA needs must be in: lgkmcnt(rb x blocks read after it)
        seq = [rd for n in range(len(self.order)) for rd in reads.get(n, [])]
        need = max(seq.index(("am", 0)), max(seq.index(("bn", j)) for j in range(self.bn - 1)))
        self.lgk_start = min(15, self.rb * (len(seq) - 1 - need))
        assert seq[-1][0] == "am" and seq[-2] == ("bn", self.bn - 1)   # lgkmcnt(rb) before MFMA bn - 1
        # LDS-DMA after the barrier (second half): every MFMA gap from the barrier's on, one or two
        # loads each
        free = list(range(self.barrier_after, len(self.order)))
        per, extra = divmod(self.loads, len(free))
        plan, k = {}, 0
        for q, n in enumerate(free):
            cnt = per + (1 if q < extra else 0)
            plan[n] = list(range(k, k + cnt))
            k += cnt
        assert k == self.loads and max(len(v) for v in plan.values()) <= 2
        self.dma_plan = plan
        self.setup_after = (0, 1, 2)
        assert max(self.setup_after) <= self.barrier_after < self.bn - 1
        assert self.epi_x >= 28 and self.vop0 % 2 == 0 and self.e_stores + self.loads <= 63
        assert self.vop0 + 56 <= self.vacc0          # the epilogue's other temporaries (up to vop0 + 55)
        assert self.nl * 4 * 1024 == KKS * tm and self.nr * 4 * 1024 == KKS * tn
        assert KSLOTS * self.slot + 16384 <= 160 * 1024   # two slots and the schedule tables

    def read_base(self, side, b):
        raise NotImplementedError


KCONFIGS = (KConfig(256, 320, False), KConfig(256, 320, True))
SGPR_K = dict(SGPR, RECA=SGPR["CM0"], RECB=SGPR["CN0"], HALF="s89")


class GenK(Gen):
    """The K-major pipeline; the bf16 epilogue (and vm model) is the wgrad kernels'."""

    def wait_oldest(self):
        s, OP, c = SGPR_K, self.OP, self.cfg
        self.emit(f"s_sub_u32 {s['NEED']}, {OP['vmt']}, {OP['q0']}")
        self.emit(f"s_mov_b32 {OP['q0']}, {OP['q1']}")
        self.emit(f"s_mov_b32 {OP['q1']}, {OP['q2']}")
        self.emit(f"s_sub_u32 {OP['np']}, {OP['np']}, 1")
        # after the oldest stage: nothing (a stage's barrier), or at a tile's start the previous
        # epilogue's stores and / or the stage the tile's top-up issued
        counts = sorted({c.e_stores + c.loads, c.e_stores, c.loads}, reverse=True)
        done = self.label("wdone")
        tgt = {n: self.label(f"w{n}_") for n in counts}
        for n in counts:
            self.emit(f"s_cmp_ge_u32 {s['NEED']}, {n}")
            self.emit(f"s_cbranch_scc1 {tgt[n]}")
        self.emit("s_waitcnt vmcnt(0)")
        self.emit(f"s_branch {done}")
        for n in counts:
            self.emit(f"{tgt[n]}:")
            self.emit(f"s_waitcnt vmcnt({n})")
            self.emit(f"s_branch {done}")
        self.emit(f"{done}:")

    def issue_setup(self):
        """Buffer resources of the cursor's stage: base at its K offset, num_records ending at the
        last valid row's K bytes of the stage (rows past the group end / N, and a half stage's
        second half of the last valid row, read as zero); this wave's LDS-DMA base in slot ISLOT."""
        s, OP, e = SGPR_K, self.OP, self.emit
        e(f"s_min_i32 {s['T']}, {s['REM']}, {KKS}")
        e(f"s_max_i32 {s['T']}, {s['T']}, 0")
        e(f"s_add_u32 {s['RL2']}, {s['RECA']}, {s['T']}")
        e(f"s_add_u32 {s['RR2']}, {s['RECB']}, {s['T']}")
        e(f"s_mov_b32 {s['RL0']}, {s['BL0']}")
        e(f"s_and_b32 {s['RL1']}, {s['BL1']}, 0xffff")
        e(f"s_mov_b32 {s['RL3']}, 0x{WORD3:x}")
        e(f"s_mov_b32 {s['RR0']}, {s['BR0']}")
        e(f"s_and_b32 {s['RR1']}, {s['BR1']}, 0xffff")
        e(f"s_mov_b32 {s['RR3']}, 0x{WORD3:x}")
        e(f"s_add_u32 {s['IB']}, {OP['lds_base']}, {s['ISLOT']}")
        e(f"s_add_u32 {s['IB']}, {s['IB']}, {OP['w1k']}")

    def issue_finish(self):
        s, OP, e, c = SGPR_K, self.OP, self.emit, self.cfg
        e(f"s_add_u32 {OP['vmt']}, {OP['vmt']}, {c.loads}")
        for n, q in enumerate(("q0", "q1", "q2")):
            e(f"s_cmp_eq_u32 {OP['np']}, {n}")
            e(f"s_cselect_b32 {OP[q]}, {OP['vmt']}, {OP[q]}")
        e(f"s_add_u32 {OP['np']}, {OP['np']}, 1")
        e(f"s_add_u32 {s['IDX']}, {s['IDX']}, 1")
        e(f"s_sub_i32 {s['REM']}, {s['REM']}, {KKS}")
        e(f"s_add_u32 {s['BL0']}, {s['BL0']}, {KKS}")
        e(f"s_addc_u32 {s['BL1']}, {s['BL1']}, 0")
        e(f"s_add_u32 {s['BR0']}, {s['BR0']}, {KKS}")
        e(f"s_addc_u32 {s['BR1']}, {s['BR1']}, 0")
        e(f"s_sub_u32 {s['ISLOT']}, {c.slot}, {s['ISLOT']}")

    def cursor_prep(self):
        """Move the cursor to the next tile once this one is fully issued (the next tile's first
        stage is its limit there: the other slot stages this tile's epilogue); SCC = a stage to
        issue."""
        s, OP, e = SGPR_K, self.OP, self.emit
        nosw = self.label("nosw")
        e(f"s_cmp_eq_u32 {s['INT']}, 1")
        e(f"s_cbranch_scc0 {nosw}")
        e(f"s_cmp_eq_u32 {s['IDX']}, {s['S']}")
        e(f"s_cbranch_scc0 {nosw}")
        e(f"s_mov_b32 {s['INT']}, 0")
        e(f"s_mov_b32 {s['IDX']}, 0")
        e(f"s_mov_b32 {s['REM']}, {OP['klenN']}")
        e(f"s_add_u32 {s['T']}, {OP['klenN']}, {KKS - 1}")
        e(f"s_lshr_b32 {s['T']}, {s['T']}, 7")
        e(f"s_min_u32 {s['LIM']}, {s['T']}, 1")
        e(f"s_mov_b32 {s['BL0']}, {OP['bLN_lo']}")
        e(f"s_mov_b32 {s['BL1']}, {OP['bLN_hi']}")
        e(f"s_mov_b32 {s['BR0']}, {OP['bRN_lo']}")
        e(f"s_mov_b32 {s['BR1']}, {OP['bRN_hi']}")
        e(f"s_mov_b32 {s['RECA']}, {OP['recAN']}")
        e(f"s_mov_b32 {s['RECB']}, {OP['recBN']}")
        e(f"{nosw}:")
        e(f"s_cmp_lt_u32 {s['IDX']}, {s['LIM']}")

    def read_block(self, side, b, slot, kh=0):
        """Block b of one side for K-half kh: two 128-bit reads (logical chunks 4 kh + 2 h and
        4 kh + 2 h + 1 of row l % 32, h = l / 32) from slot `slot`."""
        c, e = self.cfg, self.emit
        reg0 = c.am(b) if side == "am" else c.bn_reg(b)
        off = 4096 * b                  # 32 rows of 128 bytes; the side's offset is in the base
        for hh, hl in enumerate(("lo", "hi")):
            e(f"v_add_u32 {c.vt}, {slot}, {self.OP[f'{side}{hl}{kh}']}")
            e(f"ds_read_b128 v[{reg0 + 4 * hh}:{reg0 + 4 * hh + 3}], {c.vt} offset:{off}")

    def mfma(self, i, j, first):
        c = self.cfg
        d = c.acc_range(i, j)
        src = "0" if first else d
        a, b = c.bn_reg(j), c.am(i)
        self.emit(f"v_mfma_f32_32x32x64_f8f6f4 {d}, v[{a}:{a + 7}], v[{b}:{b + 7}], {src}"
                  + (" blgp:1" if c.a_e5m2 else ""))

    def half(self, kh, first, wait_first, barrier, reads_from, issue):
        """One K-half: 4 x 5 MFMAs. wait_first: the half's operands were read by the tile's
        prologue (all in); barrier: wait for the next stage's loads and pass the barrier after
        MFMA barrier_after; reads_from: (slot register, K-half) of the next half's operands, or None;
        issue: the cursor's next stage goes out after the barrier."""
        s, e, c = SGPR_K, self.emit, self.cfg
        setup = self.capture(self.issue_setup) if issue else []
        third = (len(setup) + 2) // 3
        pieces = [setup[:third], setup[third:2 * third], setup[2 * third:]]
        e("s_waitcnt lgkmcnt(0)" if wait_first else f"s_waitcnt lgkmcnt({c.lgk_start})")
        for n, (i, j) in enumerate(c.order):
            if not wait_first and n == c.bn - 1:
                e(f"s_waitcnt lgkmcnt({c.rb})")
            self.mfma(i, j, first)
            if issue and n in c.setup_after:
                for line in pieces[c.setup_after.index(n)]:
                    e(line)
            if n == c.barrier_after:
                e("s_waitcnt lgkmcnt(0)")
                if barrier:
                    self.wait_oldest()
                    e("s_barrier")
            if reads_from is not None:
                for side, b in c.reads_after.get(n, []):
                    self.read_block(side, b, reads_from[0], reads_from[1])
            if issue and n in c.dma_plan:
                for k in c.dma_plan[n]:
                    self.issue_dma(k)
                    if k == c.loads - 1:
                        self.issue_finish()

    def kstage(self, first, last, issue, half_only=False):
        """Stage k from slot CS: K-half 0 (reading half 1 from CS), then K-half 1 (unless last:
        barrier after its third MFMA, then reading the next stage's half 0 from NS = the other
        slot, and with issue the cursor's next stage into CS). half_only: the tile's last stage
        under K % 128 == 64, half 0 alone."""
        s, e, c = SGPR_K, self.emit, self.cfg
        assert not (half_only and not last) and not (issue and last)
        if not last:
            e(f"s_sub_u32 {s['NS']}, {c.slot}, {s['CS']}")
        self.half(0, first, first, False, None if half_only else (s["CS"], 1), False)
        if half_only:
            return
        self.half(1, False, False, not last, None if last else (s["NS"], 0), issue)

    def variant_pair(self, first):
        e = self.emit
        noiss, join = self.label("noiss"), self.label("join")
        self.cursor_prep()
        e(f"s_cbranch_scc0 {noiss}")
        self.kstage(first=first, last=False, issue=True)
        e(f"s_branch {join}")
        e(f"{noiss}:")
        self.kstage(first=first, last=False, issue=False)
        e(f"{join}:")

    def last_stage(self, first):
        e = self.emit
        full, join = self.label("full"), self.label("ljoin")
        e(f"s_cmp_eq_u32 {SGPR_K['HALF']}, 0")
        e(f"s_cbranch_scc1 {full}")
        self.kstage(first=first, last=True, issue=False, half_only=True)
        e(f"s_branch {join}")
        e(f"{full}:")
        self.kstage(first=first, last=True, issue=False)
        e(f"{join}:")

    def tile(self):
        s, OP, e, c = SGPR_K, self.OP, self.emit, self.cfg
        e("s_nop 4")   # inputs may come from v_readfirstlane (VALU-written SGPRs) just before
        e(f"s_add_u32 {s['S']}, {OP['klenT']}, {KKS - 1}")
        e(f"s_lshr_b32 {s['S']}, {s['S']}, 7")
        e(f"s_and_b32 {s['HALF']}, {OP['klenT']}, {KKS // 2}")
        e(f"s_mul_i32 {s['CS']}, {OP['c0']}, {c.slot}")
        e(f"s_add_u32 {s['T']}, {OP['c0']}, {OP['nis']}")
        e(f"s_cmp_ge_u32 {s['T']}, {KSLOTS}")
        e(f"s_cselect_b32 {s['T2']}, {KSLOTS}, 0")
        e(f"s_sub_u32 {s['T']}, {s['T']}, {s['T2']}")
        e(f"s_mul_i32 {s['ISLOT']}, {s['T']}, {c.slot}")
        e(f"s_mov_b32 {s['INT']}, 1")
        e(f"s_mov_b32 {s['IDX']}, {OP['nis']}")
        e(f"s_mov_b32 {s['LIM']}, {s['S']}")
        e(f"s_lshl_b32 {s['T']}, {OP['nis']}, 7")
        e(f"s_sub_i32 {s['REM']}, {OP['klenT']}, {s['T']}")
        e(f"s_add_u32 {s['BL0']}, {OP['bLT_lo']}, {s['T']}")
        e(f"s_addc_u32 {s['BL1']}, {OP['bLT_hi']}, 0")
        e(f"s_add_u32 {s['BR0']}, {OP['bRT_lo']}, {s['T']}")
        e(f"s_addc_u32 {s['BR1']}, {OP['bRT_hi']}, 0")
        e(f"s_mov_b32 {s['RECA']}, {OP['recAT']}")
        e(f"s_mov_b32 {s['RECB']}, {OP['recBT']}")
        e("s_barrier")   # the previous tile's epilogue is done with its staging slot
        e(f"s_min_u32 {s['LIMTOP']}, {s['S']}, {KSLOTS}")
        top, topdone = self.label("top"), self.label("topdone")
        e(f"{top}:")
        e(f"s_cmp_lt_u32 {s['IDX']}, {s['LIMTOP']}")
        e(f"s_cbranch_scc0 {topdone}")
        self.issue_core()
        e(f"s_branch {top}")
        e(f"{topdone}:")
        self.wait_oldest()
        e("s_barrier")
        for i in range(c.bm):
            self.read_block("am", i, s["CS"], 0)
        for j in range(c.bn):
            self.read_block("bn", j, s["CS"], 0)
        first_last, loop, steady_last, epi = (self.label(x) for x in ("fl", "loop", "sl", "epi"))
        e(f"s_cmp_eq_u32 {s['S']}, 1")
        e(f"s_cbranch_scc1 {first_last}")
        self.variant_pair(first=True)
        e(f"s_mov_b32 {s['CS']}, {s['NS']}")
        e(f"s_mov_b32 {s['K']}, 1")
        e(f"{loop}:")
        e(f"s_add_u32 {s['T']}, {s['K']}, 1")
        e(f"s_cmp_eq_u32 {s['T']}, {s['S']}")
        e(f"s_cbranch_scc1 {steady_last}")
        self.variant_pair(first=False)
        e(f"s_mov_b32 {s['CS']}, {s['NS']}")
        e(f"s_add_u32 {s['K']}, {s['K']}, 1")
        e(f"s_branch {loop}")
        e(f"{first_last}:")
        self.last_stage(first=True)
        e(f"s_branch {epi}")
        e(f"{steady_last}:")
        self.last_stage(first=False)
        e(f"{epi}:")
        self.epilogue()
        e(f"s_cmp_eq_u32 {s['INT']}, 0")
        e(f"s_cselect_b32 {OP['nis']}, {s['IDX']}, 0")


def render():
    out = ["// Generated by gen_vark_wide.py; do not edit. Per-tile bodies of the wide-tile FP8 grouped",
           "// wgrad kernels (vark_wide.h) and of the wide persistent fwd / dgrad kernel (persistent_wide.h):",
           "// gfx950 assembly, one inline asm statement per tile shape."]
    total = 0
    for c in CONFIGS + KCONFIGS:
        g = GenK(c) if isinstance(c, KConfig) else Gen(c)
        g.tile()
        total += len(g.lines)
        text = "\\n\\t".join(g.lines)
        clob = ([f'"a{r}"' for r in range(256)] + [f'"v{r}"' for r in c.vgpr_clobber]
                + [f'"s{r}"' for r in c.sgpr_clobber] + ['"m0"', '"scc"', '"memory"'])
        order = ", ".join(f"{i}:{n}" for i, (n, _) in enumerate(c.operands))
        t = c.name
        out += [
            f"// {t} operands: {order}",
            f"#define GGEMM_WIDE_NOPERANDS_{t} {len(c.operands)}",
            f"#define GGEMM_WIDE_E_STORES_{t} {c.e_stores}",
            f"#define GGEMM_WIDE_ASM_{t} \"{text}\"",
            f"#define GGEMM_WIDE_CLOBBERS_{t} " + ", ".join(clob),
        ]
    return "\n".join(out) + "\n", total


def main(path=OUT):
    text, n = render()
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)
    return n


if __name__ == "__main__":
    print(f"{main(sys.argv[1] if len(sys.argv) > 1 else OUT)} instructions and labels")
