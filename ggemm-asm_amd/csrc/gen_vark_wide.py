#!/usr/bin/env python3
"""Writes vark_wide_asm.inc: the per-tile body of the wide-tile FP8 grouped wgrad kernel
(vark_wide.h) as one gfx950 inline-assembly statement.

Why assembly: a 256 x 384 output tile on four waves (one per SIMD) needs 384 fp32 accumulators
per wave, 256 in AGPRs and 128 in VGPRs. The compiler gives every MFMA of a kernel the same
accumulator register class (at most 256 AGPRs), so it cannot build this kernel without spilling;
written out here, the accumulators sit in fixed registers for the whole K loop.

One statement computes one tile of one group (the HIP code around it walks the schedule, see
vark_wide.h) and keeps the operand pipeline running across tiles:
  * the token axis in stages of 64: LDS holds three stage slots of 40 KiB (64 rows of 256 LHS
    bytes, then 64 rows of 384 RHS bytes), filled by LDS-DMA (buffer_load_dwordx4 ... lds, 1 KiB per
    wave-instruction, 4 LHS + 6 RHS per wave and stage), bounded by the buffer's num_records so
    tokens past the group end read as zero;
  * an issue cursor walks this tile's stages, then the next tile's first two: at each stage's
    barrier the slot just released takes the cursor's next stage, so up to three stages are in
    flight; counted vmcnt waits use a per-wave model of outstanding vector-memory operations
    (in/out operands, so it survives between tiles);
  * per stage and wave 24 v_mfma_f32_32x32x64_f8f6f4 (4 LHS blocks x 6 RHS blocks of 32, A = RHS
    e5m2 with cbsz 1, B = LHS e4m3), operands read with ds_read_b64_tr_b8 as the MFMAs release
    their registers, the barrier that publishes the next stage placed after the first column;
  * the epilogue scales by s_lhs * s_rhs, converts to bf16 (RNE), stages each 32 x 64 piece
    through the freed slot (XOR swizzle, conflict-free) and stores whole 128-byte row segments
    non-temporally; rows past OUT_M fall outside the C buffer resource and are dropped.

Operands (numbered as the asm statement in vark_wide.h passes them) are listed in OPERANDS; run
this script to rewrite the include after changing it (build.py runs it before every build).
"""
from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "vark_wide_asm.inc")

SLOT = 40960                 # bytes per stage slot
SLOTS = 3
RHS_OFF = 16384              # RHS rows follow 64 rows of 256 LHS bytes
WORD3 = 0x00020000           # raw buffer resource word 3 (32-bit data format)
E_STORES = 48                # C stores per wave and tile (12 passes x 4)
LOADS = 10                   # LDS-DMA instructions per wave and stage

# in/out ("+s") then inputs: (name, constraint)
OPERANDS = [
    ("c0", "+s"), ("nis", "+s"), ("vmt", "+s"), ("q0", "+s"), ("q1", "+s"), ("q2", "+s"), ("np", "+s"),
    ("lds_base", "s"), ("w1k", "s"),
    ("bLT_lo", "s"), ("bLT_hi", "s"), ("bRT_lo", "s"), ("bRT_hi", "s"), ("klenT", "s"), ("m0T", "s"), ("n0T", "s"),
    ("bLN_lo", "s"), ("bLN_hi", "s"), ("bRN_lo", "s"), ("bRN_hi", "s"), ("klenN", "s"), ("m0N", "s"), ("n0N", "s"),
    ("cT_lo", "s"), ("cT_hi", "s"), ("crecT", "s"),
    ("stride_l", "s"), ("stride_r", "s"), ("cm2", "s"), ("alpha", "s"), ("sw_epi", "s"),
    ("voffL0", "v"), *[(f"voffR{j}", "v") for j in range(6)], *[(f"amb{i}", "v") for i in range(4)],
    *[(f"bnb{j}", "v") for j in range(6)], ("ew_base", "v"), ("ew_s", "v"), ("rb_even", "v"), ("rb_odd", "v"),
    ("gb", "v"),
]
OP = {name: f"%{i}" for i, (name, _) in enumerate(OPERANDS)}

# scalar temporaries (clobbered): buffer resources in aligned quads, then state
SGPR = dict(
    RL="s[56:59]", RL0="s56", RL1="s57", RL2="s58", RL3="s59",
    RR="s[60:63]", RR0="s60", RR1="s61", RR2="s62", RR3="s63",
    RC="s[64:67]", RC0="s64", RC1="s65", RC2="s66", RC3="s67",
    S="s68", K="s69", INT="s70", IDX="s71", REM="s72", LIM="s73",
    BL0="s74", BL1="s75", BR0="s76", BR1="s77", CM0="s78", CN0="s79",
    ISLOT="s80", CS="s81", NS="s82", T="s83", T2="s84", L16="s85", NEED="s86", LIMTOP="s87", EPI="s88",
    IB="s89",
)
SGPR_CLOBBER = list(range(56, 90))
VGPR_CLOBBER = list(range(36, 256))      # v36-v47 temps, v48-v127 operands, v128-v255 accumulators
VT, VT2 = "v36", "v37"                   # address temporaries


def acc(i, j):
    """Accumulator registers of block (m-block i, n-block j): blocks 0-15 in AGPRs, 16-23 in VGPRs."""
    b = 6 * i + j
    if b < 16:
        return "a", 16 * b
    return "v", 128 + 16 * (b - 16)


def acc_range(i, j):
    kind, base = acc(i, j)
    return f"{kind}[{base}:{base + 15}]"


def am(i):
    return 48 + 8 * i


def bn(j):
    return 80 + 8 * j


class Gen:
    def __init__(self):
        self.lines = []
        self.nlabel = 0

    def emit(self, s):
        self.lines.append(s)

    def label(self, stem):
        self.nlabel += 1
        return f".Lggw_{stem}{self.nlabel}_%="

    # ---------------------------------------------------------------- vm model

    def wait_oldest(self):
        """Wait for the oldest issued, not yet awaited stage; pop it from the model. vmcnt is
        rounded down to one of the counts this kernel can produce (a stricter wait is safe)."""
        s = SGPR
        self.emit(f"s_sub_u32 {s['NEED']}, {OP['vmt']}, {OP['q0']}")
        self.emit(f"s_mov_b32 {OP['q0']}, {OP['q1']}")
        self.emit(f"s_mov_b32 {OP['q1']}, {OP['q2']}")
        self.emit(f"s_sub_u32 {OP['np']}, {OP['np']}, 1")
        counts = [E_STORES + LOADS, E_STORES, 2 * LOADS, LOADS]
        done = self.label("wdone")
        tgt = {c: self.label(f"w{c}_") for c in counts}
        self.emit(f"s_cmp_eq_u32 {s['NEED']}, {LOADS}")        # the steady state: one stage behind
        self.emit(f"s_cbranch_scc1 {tgt[LOADS]}")
        for c in counts:
            self.emit(f"s_cmp_ge_u32 {s['NEED']}, {c}")
            self.emit(f"s_cbranch_scc1 {tgt[c]}")
        self.emit("s_waitcnt vmcnt(0)")
        self.emit(f"s_branch {done}")
        for c in counts:
            self.emit(f"{tgt[c]}:")
            self.emit(f"s_waitcnt vmcnt({c})")
            self.emit(f"s_branch {done}")
        self.emit(f"{done}:")

    # ---------------------------------------------------------------- issue

    def capture(self, fn, *args):
        """The lines fn would emit, without emitting them."""
        saved, self.lines = self.lines, []
        fn(*args)
        out, self.lines = self.lines, saved
        return out

    def issue_setup(self):
        """Buffer resources of the cursor's stage and this wave's LDS-DMA base in slot ISLOT."""
        s = SGPR
        e = self.emit
        e(f"s_min_i32 {s['T']}, {s['REM']}, 64")
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

    def issue_dma(self, j):
        """LDS-DMA instruction j of the stage (0-3: LHS rows, 4-9: RHS rows)."""
        s = SGPR
        e = self.emit
        if j < 4:
            e(f"s_add_u32 m0, {s['IB']}, {4096 * j}")
            if j == 0:
                e("s_nop 0")
                e(f"buffer_load_dwordx4 {OP['voffL0']}, {s['RL']}, 0 offen lds")
            else:
                e(f"s_mul_i32 {s['T2']}, {s['L16']}, {j}")
                e(f"v_add_u32 {VT2}, {s['T2']}, {OP['voffL0']}")
                e(f"buffer_load_dwordx4 {VT2}, {s['RL']}, 0 offen lds")
        else:
            jj = j - 4
            e(f"s_add_u32 m0, {s['IB']}, {RHS_OFF + 4096 * jj}")
            e("s_nop 0")
            e(f"buffer_load_dwordx4 {OP[f'voffR{jj}']}, {s['RR']}, 0 offen lds")

    def issue_finish(self):
        """Model: LOADS more operations, the count right after this stage remembered; advance the
        cursor to its next stage and slot."""
        s = SGPR
        e = self.emit
        e(f"s_add_u32 {OP['vmt']}, {OP['vmt']}, {LOADS}")
        for n, q in enumerate(("q0", "q1", "q2")):
            e(f"s_cmp_eq_u32 {OP['np']}, {n}")
            e(f"s_cselect_b32 {OP[q]}, {OP['vmt']}, {OP[q]}")
        e(f"s_add_u32 {OP['np']}, {OP['np']}, 1")
        e(f"s_add_u32 {s['IDX']}, {s['IDX']}, 1")
        e(f"s_sub_i32 {s['REM']}, {s['REM']}, 64")
        e(f"s_lshl_b32 {s['T']}, {OP['stride_l']}, 6")
        e(f"s_add_u32 {s['BL0']}, {s['BL0']}, {s['T']}")
        e(f"s_addc_u32 {s['BL1']}, {s['BL1']}, 0")
        e(f"s_lshl_b32 {s['T']}, {OP['stride_r']}, 6")
        e(f"s_add_u32 {s['BR0']}, {s['BR0']}, {s['T']}")
        e(f"s_addc_u32 {s['BR1']}, {s['BR1']}, 0")
        e(f"s_add_u32 {s['ISLOT']}, {s['ISLOT']}, {SLOT}")
        e(f"s_cmp_ge_u32 {s['ISLOT']}, {SLOT * SLOTS}")
        e(f"s_cselect_b32 {s['T']}, {SLOT * SLOTS}, 0")
        e(f"s_sub_u32 {s['ISLOT']}, {s['ISLOT']}, {s['T']}")

    def issue_core(self):
        """Issue the cursor's stage into slot ISLOT and advance the cursor."""
        self.issue_setup()
        for j in range(LOADS):
            self.issue_dma(j)
        self.issue_finish()

    def cursor_prep(self):
        """Before a stage that may issue: move the cursor to the next tile once this one is fully
        issued (the next tile's first two stages are the cursor's limit there); SCC = the cursor
        has a stage to issue."""
        s = SGPR
        e = self.emit
        nosw = self.label("nosw")
        e(f"s_cmp_eq_u32 {s['INT']}, 1")
        e(f"s_cbranch_scc0 {nosw}")
        e(f"s_cmp_eq_u32 {s['IDX']}, {s['S']}")
        e(f"s_cbranch_scc0 {nosw}")
        e(f"s_mov_b32 {s['INT']}, 0")
        e(f"s_mov_b32 {s['IDX']}, 0")
        e(f"s_mov_b32 {s['REM']}, {OP['klenN']}")
        e(f"s_add_u32 {s['T']}, {OP['klenN']}, 63")
        e(f"s_lshr_b32 {s['T']}, {s['T']}, 6")
        e(f"s_min_u32 {s['LIM']}, {s['T']}, 2")
        e(f"s_mov_b32 {s['BL0']}, {OP['bLN_lo']}")
        e(f"s_mov_b32 {s['BL1']}, {OP['bLN_hi']}")
        e(f"s_mov_b32 {s['BR0']}, {OP['bRN_lo']}")
        e(f"s_mov_b32 {s['BR1']}, {OP['bRN_hi']}")
        e(f"s_mov_b32 {s['CM0']}, {OP['m0N']}")
        e(f"s_mov_b32 {s['CN0']}, {OP['n0N']}")
        e(f"{nosw}:")
        e(f"s_cmp_lt_u32 {s['IDX']}, {s['LIM']}")

    # ---------------------------------------------------------------- operands

    def read_am(self, i, slot):
        e = self.emit
        e(f"v_add_u32 {VT}, {slot}, {OP[f'amb{i}']}")
        for n, off in enumerate((0, 8 * 256, 32 * 256, 40 * 256)):
            r = am(i) + 2 * n
            e(f"ds_read_b64_tr_b8 v[{r}:{r + 1}], {VT} offset:{off}")

    def read_bn(self, j, slot):
        e = self.emit
        e(f"v_add_u32 {VT}, {slot}, {OP[f'bnb{j}']}")
        for n, off in enumerate((0, 8 * 384, 32 * 384, 40 * 384)):
            r = bn(j) + 2 * n
            e(f"ds_read_b64_tr_b8 v[{r}:{r + 1}], {VT} offset:{off}")

    def mfma(self, i, j, first):
        d = acc_range(i, j)
        c = "0" if first else d
        self.emit(f"v_mfma_f32_32x32x64_f8f6f4 {d}, v[{bn(j)}:{bn(j) + 7}], v[{am(i)}:{am(i) + 7}], {c} cbsz:1")

    # ---------------------------------------------------------------- one stage

    # MFMA order within a stage: m-block 0 across all six n-blocks first, then the other three
    # m-blocks column by column. m-block 0's registers free up after six MFMAs and the n-blocks'
    # after their column, so the next stage's operands are read spread over the stage; the next
    # stage begins with m-block 0, whose operands were read earliest.
    ORDER = [(0, j) for j in range(6)] + [(i, j) for j in range(6) for i in (1, 2, 3)]
    BARRIER_AFTER = 4                                   # MFMA index after which the barrier sits
    READS_AFTER = {5: [("am", 0)], 8: [("bn", 0)], 11: [("bn", 1)], 14: [("bn", 2)], 17: [("bn", 3)],
                   20: [("bn", 4)], 21: [("am", 1)], 22: [("am", 2)], 23: [("bn", 5), ("am", 3)]}
    DMA_AFTER = [6, 7, 9, 10, 12, 13, 15, 16, 18, 19]   # LDS-DMA instruction j after MFMA DMA_AFTER[j]
    SETUP_AFTER = (0, 1, 2)                             # buffer resources, in three pieces
    FINISH_AFTER = 20

    def stage(self, first, last, issue):
        """Stage k: its operands are in registers (read during stage k-1, or at tile entry for the
        first stage); CS = its slot. Unless last: after MFMA 4 every read of slot CS has completed,
        the wave waits for stage k+1's loads and passes the barrier (stage k+1 published, slot CS
        free); stage k+1's operands are then read as their registers free up, and with issue the
        cursor's next stage goes into slot CS one LDS-DMA instruction per MFMA gap."""
        s = SGPR
        e = self.emit
        if not last:
            e(f"s_add_u32 {s['NS']}, {s['CS']}, {SLOT}")
            e(f"s_cmp_ge_u32 {s['NS']}, {SLOT * SLOTS}")
            e(f"s_cselect_b32 {s['T']}, {SLOT * SLOTS}, 0")
            e(f"s_sub_u32 {s['NS']}, {s['NS']}, {s['T']}")
        setup = self.capture(self.issue_setup) if issue else []
        pieces = [setup[:5], setup[5:10], setup[10:]]
        e("s_waitcnt lgkmcnt(0)" if first else "s_waitcnt lgkmcnt(15)")
        for n, (i, j) in enumerate(self.ORDER):
            if not first:
                # previous stage's reads ended ... bn4, am1, am2, bn5, am3 (4 reads each)
                if n == 5:
                    e("s_waitcnt lgkmcnt(4)")
            self.mfma(i, j, first)
            if issue and n in self.SETUP_AFTER:
                for line in pieces[self.SETUP_AFTER.index(n)]:
                    e(line)
            if n == self.BARRIER_AFTER:
                # every read of slot CS (this stage's operands) has completed in this wave
                e("s_waitcnt lgkmcnt(0)")
                if not last:
                    self.wait_oldest()
                    e("s_barrier")
            if last:
                continue
            for kind, b in self.READS_AFTER.get(n, []):
                (self.read_am if kind == "am" else self.read_bn)(b, s["NS"])
            if issue and n in self.DMA_AFTER:
                self.issue_dma(self.DMA_AFTER.index(n))
            if issue and n == self.FINISH_AFTER:
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
        s = SGPR
        e = self.emit
        e(f"s_mov_b32 {s['RC0']}, {OP['cT_lo']}")
        e(f"s_and_b32 {s['RC1']}, {OP['cT_hi']}, 0xffff")
        e(f"s_mov_b32 {s['RC2']}, {OP['crecT']}")
        e(f"s_mov_b32 {s['RC3']}, 0x{WORD3:x}")

    def store_offset(self, i, k, p):
        """T = this wave's byte offset of tile rows 128 wm + 32 i + 8 k, columns 192 wn + 64 p."""
        s = SGPR
        e = self.emit
        e(f"s_mul_i32 {s['T']}, {OP['cm2']}, {32 * i + 8 * k}")
        e(f"s_add_u32 {s['T']}, {s['T']}, {OP['sw_epi']}")
        if p:
            e(f"s_add_u32 {s['T']}, {s['T']}, {128 * p}")
        e(f"v_add_u32 {VT2}, {s['T']}, {OP['gb']}")

    def epilogue(self):
        s = SGPR
        e = self.emit
        e("s_nop 7")
        e("s_nop 7")
        e("s_nop 7")
        e("s_barrier")   # every wave is past its reads of the last stage's slot
        e(f"s_add_u32 {s['EPI']}, {OP['lds_base']}, {s['CS']}")
        e(f"s_lshl_b32 {s['T']}, {OP['w1k']}, 2")
        e(f"s_add_u32 {s['EPI']}, {s['EPI']}, {s['T']}")
        # staging write addresses of chunk c = 4 jj + g: row l % 32, chunk c ^ swz, half l / 32
        for c in range(8):
            e(f"v_xor_b32 v38, {c}, {OP['ew_s']}")
            e("v_lshlrev_b32 v38, 4, v38")
            e(f"v_add3_u32 v{112 + c}, v38, {OP['ew_base']}, {s['EPI']}")
        e(f"v_add_u32 v120, {s['EPI']}, {OP['rb_even']}")
        e(f"v_add_u32 v121, {s['EPI']}, {OP['rb_odd']}")
        self.c_resource()
        npass = 0
        for i in range(4):
            for p in range(3):
                dbase = 80 if npass % 2 == 0 else 96
                npass += 1
                for jj in range(2):
                    j = 2 * p + jj
                    kind, base = acc(i, j)
                    for g in range(4):
                        src = []
                        for r in range(4):
                            reg = base + 4 * g + r
                            if kind == "a":
                                e(f"v_accvgpr_read_b32 v{40 + r}, a{reg}")
                                src.append(f"v{40 + r}")
                            else:
                                src.append(f"v{reg}")
                        for r in range(4):
                            e(f"v_mul_f32 v{44 + r}, {OP['alpha']}, {src[r]}")
                        e("v_cvt_pk_bf16_f32 v38, v44, v45")
                        e("v_cvt_pk_bf16_f32 v39, v46, v47")
                        e(f"ds_write_b64 v{112 + 4 * jj + g}, v[38:39]")
                for k in range(4):
                    base_v = "v120" if k % 2 == 0 else "v121"
                    off = 2048 if k >= 2 else 0
                    d = dbase + 4 * k
                    e(f"ds_read_b128 v[{d}:{d + 3}], {base_v} offset:{off}")
                e("s_waitcnt lgkmcnt(0)")
                for k in range(4):
                    d = dbase + 4 * k
                    self.store_offset(i, k, p)
                    e(f"buffer_store_dwordx4 v[{d}:{d + 3}], {VT2}, {s['RC']}, 0 offen nt")
        e(f"s_add_u32 {OP['vmt']}, {OP['vmt']}, {E_STORES}")

    def zero_epilogue(self):
        """A tile without tokens: zeros straight from registers, the same 48 stores per wave."""
        e = self.emit
        for r in range(80, 84):
            e(f"v_mov_b32 v{r}, 0")
        self.c_resource()
        for i in range(4):
            for p in range(3):
                for k in range(4):
                    self.store_offset(i, k, p)
                    e(f"buffer_store_dwordx4 v[80:83], {VT2}, {SGPR['RC']}, 0 offen nt")
        e(f"s_add_u32 {OP['vmt']}, {OP['vmt']}, {E_STORES}")

    # ---------------------------------------------------------------- whole tile

    def tile(self):
        s = SGPR
        e = self.emit
        e("s_nop 4")   # inputs may come from v_readfirstlane (VALU-written SGPRs) just before
        e(f"s_add_u32 {s['S']}, {OP['klenT']}, 63")
        e(f"s_lshr_b32 {s['S']}, {s['S']}, 6")
        e(f"s_lshl_b32 {s['L16']}, {OP['stride_l']}, 4")
        e(f"s_mul_i32 {s['CS']}, {OP['c0']}, {SLOT}")
        e(f"s_add_u32 {s['T']}, {OP['c0']}, {OP['nis']}")
        e(f"s_cmp_ge_u32 {s['T']}, {SLOTS}")
        e(f"s_cselect_b32 {s['T2']}, {SLOTS}, 0")
        e(f"s_sub_u32 {s['T']}, {s['T']}, {s['T2']}")
        e(f"s_mul_i32 {s['ISLOT']}, {s['T']}, {SLOT}")
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
        for i in range(4):
            self.read_am(i, s["CS"])
        for j in range(6):
            self.read_bn(j, s["CS"])
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


def render():
    g = Gen()
    g.tile()
    text = "\\n\\t".join(g.lines)
    clob = ([f'"a{r}"' for r in range(256)] + [f'"v{r}"' for r in VGPR_CLOBBER]
            + [f'"s{r}"' for r in SGPR_CLOBBER] + ['"m0"', '"scc"', '"memory"'])
    order = ", ".join(f"{i}:{n}" for i, (n, _) in enumerate(OPERANDS))
    out = [
        "// Generated by gen_vark_wide.py; do not edit. Per-tile body of the wide-tile FP8 grouped",
        "// wgrad kernel (vark_wide.h): gfx950 assembly for one inline asm statement.",
        f"// Operands: {order}",
        f"#define GGEMM_WIDE_NOPERANDS {len(OPERANDS)}",
        f"#define GGEMM_WIDE_E_STORES {E_STORES}",
        f"#define GGEMM_WIDE_LOADS {LOADS}",
        f"#define GGEMM_WIDE_ASM \"{text}\"",
        "#define GGEMM_WIDE_CLOBBERS " + ", ".join(clob),
        "",
    ]
    return "\n".join(out), len(g.lines)


def main(path=OUT):
    text, n = render()
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)
    return n


if __name__ == "__main__":
    print(f"{main(sys.argv[1] if len(sys.argv) > 1 else OUT)} instructions and labels")
