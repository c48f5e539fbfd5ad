"""CPU checks of the wide persistent kernel's generated assembly (the K-major configurations of
ggemm-asm_amd/csrc/gen_vark_wide.py, persistent_wide.h), before any GPU launch.

The per-tile assembly statement runs in the scalar interpreter of test_vark_wide_host.py (SALU
arithmetic, branches, m0; vector-memory, LDS and MFMA instructions recorded as events), with the
HIP tile loop around it restated (c0 += stages mod 2, the in/out operands carried). Over tile
sequences of both K parities (K % 128 == 0 and == 64, one-stage tiles included), ragged tiles and
both formats the recorded program must:
  * issue every stage of every tile once, in order, into slot (stage index mod 2), with the buffer
    base at the stage's K offset and num_records ending at the last valid row's K bytes of the
    stage;
  * wait (counted vmcnt, in-order completion) for a stage's loads and pass a barrier before any
    wave reads it, never DMA into a slot before a barrier that follows the last reads of its
    previous stage or of the epilogue staged there, nor stage C before a barrier that follows
    every read of the tile's last stage;
  * give every MFMA, in its A and B registers, completed LDS reads of its own blocks, K-half and
    stage (in-order lgkmcnt), with a zero accumulator input exactly in a tile's first K-half, and
    the B-operand format of the A tensor;
  * store each epilogue's whole lines of the wave's quadrant, bounded by the tile's valid rows;
  * take the same branches and barriers in every wave.
Per-lane maps (DMA placement, operand reads) are checked against the 32x32x64 operand layout, the
K order both operands share, and LDS bank conflicts.
"""
import re

import numpy as np
import pytest

import test_vark_wide_host as W

GEN = W.GEN
M32 = W.M32
KCFGS = {c.name: c for c in GEN.KCONFIGS}


def _kprogram(cfg):
    g = GEN.GenK(cfg)
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


KPROGS = {name: _kprogram(c) for name, c in KCFGS.items()}


class _Events(list):
    """Event list that resolves ds_read_b128 addresses (slot value, base operand) at issue."""

    def __init__(self, blk):
        super().__init__()
        self.blk = blk

    def append(self, e):
        if e[0] == "ds_read_b128":
            reg, mod = e[1][1].split()
            off = int(mod.split(":")[1]) if ":" in mod else 0
            super().append(("read", self.blk.v[reg], off, e[1][0]))
        else:
            super().append(e)


A, B, OUT = 0x7F0000000000, 0x7E0000000000, 0x7D0000000000


def _run(cfg, tiles, K, wave, sam, sbg, sbn, scm):
    """tiles: list of (g, row0, rows, n0). Returns (events, per-tile spans, final state)."""
    ev = _Events(None)
    scal = {f"s{r}": 0 for r in cfg.sgpr_clobber}
    state = dict(c0=0, nis=0, vmt=0, q0=0, q1=0, q2=0, np=0)
    spans = []
    S = (K + 127) // 128
    for n, (g, row0, rows, n0) in enumerate(tiles):
        has_next = n + 1 < len(tiles)
        N = tiles[n + 1] if has_next else tiles[n]
        blt, brt = A + row0 * sam, B + g * sbg + n0 * sbn
        bln, brn = A + N[1] * sam, B + N[0] * sbg + N[3] * sbn
        ops = dict(state)
        ops.update(lds_base=0, w1k=1024 * wave,
                   bLT_lo=blt & M32, bLT_hi=blt >> 32, bRT_lo=brt & M32, bRT_hi=brt >> 32, klenT=K,
                   recAT=(rows - 1) * sam, recBT=(cfg.tn - 1) * sbn,
                   bLN_lo=bln & M32, bLN_hi=bln >> 32, bRN_lo=brn & M32, bRN_hi=brn >> 32,
                   klenN=K if has_next else 0, recAN=(N[2] - 1) * sam, recBN=(cfg.tn - 1) * sbn,
                   cT_lo=(OUT + 2 * (row0 * scm + n0)) & M32, cT_hi=(OUT + 2 * (row0 * scm + n0)) >> 32,
                   crecT=(rows * scm - n0) * 2, cm2=2 * scm, alpha=0x3F800000,
                   sw_epi=(32 * cfg.bm * (wave & 1) * scm + 32 * cfg.bn * (wave >> 1)) * 2)
        start = len(ev)
        blk = W.Block(cfg, ops, None, scal, KPROGS[cfg.name])
        blk.ev = ev
        ev.blk = blk
        blk.run()
        spans.append((start, len(ev)))
        for k in state:
            state[k] = ops[k]
        state["c0"] = (state["c0"] + S) % 2
    return ev, spans, state


def _regs(r):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", r)
    return list(range(int(m.group(1)), int(m.group(2)) + 1))


def _check(cfg, tiles, K, wave=0, sam=2880, sbg=5760 * 2880, sbn=2880, scm=5760):
    ev, spans, state = _run(cfg, tiles, K, wave, sam, sbg, sbn, scm)
    op = lambda name: "%" + str([n for n, _ in cfg.operands].index(name))
    S = (K + 127) // 128
    tail = K % 128 == 64
    L = cfg.loads
    stages = [(n, s) for n in range(len(tiles)) for s in range(S)]
    slot_of = {st: k % 2 for k, st in enumerate(stages)}
    # K-halves: (tile, stage, kh)
    halves = [(n, s, kh) for n in range(len(tiles)) for s in range(S) for kh in range(1 if (tail and s == S - 1) else 2)]
    # ---- DMA
    dmas = [(i, e) for i, e in enumerate(ev) if e[0] == "dma"]
    assert len(dmas) == L * len(stages)
    issue_pos = {}
    for k, (n, s) in enumerate(stages):
        g, row0, rows, n0 = tiles[n]
        grp = dmas[L * k:L * k + L]
        issue_pos[(n, s)] = (grp[0][0], grp[-1][0])
        kv = min(128, K - 128 * s)
        for j, (_, e) in enumerate(grp):
            _, m0v, (base, nrec, stride_bits, w3), voff, _ = e
            assert stride_bits == 0 and w3 == GEN.WORD3
            if j < cfg.nl:
                assert base == A + row0 * sam + 128 * s
                assert nrec == (rows - 1) * sam + kv
                assert m0v == slot_of[(n, s)] * cfg.slot + 1024 * wave + 4096 * j
                assert voff == (0, op(f"voffL{j}"))
            else:
                jj = j - cfg.nl
                assert base == B + g * sbg + n0 * sbn + 128 * s
                assert nrec == (cfg.tn - 1) * sbn + kv
                assert m0v == slot_of[(n, s)] * cfg.slot + cfg.rhs_off + 1024 * wave + 4096 * jj
                assert voff == (0, op(f"voffR{jj}"))
            assert m0v + 1024 <= GEN.KSLOTS * cfg.slot
    # ---- operand reads: 2 (bm + bn) per K-half, from the half's slot, bases of its K-half
    R = 2 * (cfg.bm + cfg.bn)
    reads = [(i, e) for i, e in enumerate(ev) if e[0] == "read" and e[1][1] in
             {op(f"{sd}{hl}{kh}") for sd in ("am", "bn") for hl in ("lo", "hi") for kh in (0, 1)}]
    assert len(reads) == R * len(halves)
    read_span, read_of = {}, {}
    for k, h in enumerate(halves):
        n, s, kh = h
        grp = reads[R * k:R * k + R]
        read_span[h] = (grp[0][0], grp[-1][0])
        want = sorted((op(f"{sd}{hl}{kh}"), 4096 * b) for sd, nb in (("am", cfg.bm), ("bn", cfg.bn))
                      for b in range(nb) for hl in ("lo", "hi"))
        got = []
        for i, (_, (slot_off, name), off, dst) in grp:
            assert slot_off == slot_of[(n, s)] * cfg.slot, (h, slot_off)
            got.append((name, off))
            read_of[i] = h
        assert sorted(got) == want
    # ---- completion model: in-order vmcnt, barriers
    issued, done_at = [], {}
    barriers = [i for i, e in enumerate(ev) if e[0] == "barrier"]
    for i, e in enumerate(ev):
        if e[0] in ("dma", "store"):
            issued.append(i)
        elif e[0] == "vmcnt":
            for op_i in issued[:max(len(issued) - e[1], 0)]:
                done_at.setdefault(op_i, i)
    for st in stages:
        first_read = read_span[(st[0], st[1], 0)][0]
        a, b = issue_pos[st]
        loads = [i for i in issued if a <= i <= b]
        assert all(i in done_at and done_at[i] < first_read for i in loads), f"stage {st} read before its loads"
        last_done = max(done_at[i] for i in loads)
        assert any(last_done < bi < first_read for bi in barriers), f"stage {st}: no barrier after its wait"
    # ---- data flow: every MFMA's registers hold completed reads of its blocks, K-half and stage;
    # no LDS load is issued into a register another LDS load still in flight writes
    pending, last = [], {}
    blk_of = {cfg.acc_range(i, j): (i, j) for i in range(cfg.bm) for j in range(cfg.bn)}
    mf_k = 0
    nblk = cfg.bm * cfg.bn
    for i, e in enumerate(ev):
        if e[0] == "read":
            rs = set(_regs(e[3]))
            assert not any(rs & p for p in pending), "two LDS loads in flight to one register"
            pending.append(rs)
            for r in rs:
                last[r] = (i, e[1], e[2])
        elif e[0] in ("ds_write_b64", "ds_write_b128"):
            pending.append(set())
        elif e[0] == "lgkmcnt":
            pending = pending[len(pending) - e[1]:] if e[1] < len(pending) else pending
        elif e[0] == "mfma":
            h = halves[mf_k // nblk]
            n, s, kh = h
            mf_k += 1
            ii, jj = blk_of[e[1]]
            a_regs, b_regs = _regs(e[2]), _regs(e[3])
            assert a_regs[0] == cfg.bn_reg(jj) and b_regs[0] == cfg.am(ii)
            assert not any(set(a_regs + b_regs) & p for p in pending), f"MFMA {e} reads a pending LDS load"
            for regs, sd, b in ((a_regs, "bn", jj), (b_regs, "am", ii)):
                for q, r in enumerate(regs):
                    ri, (slot_off, name), off = last[r]
                    assert read_of.get(ri) == h, f"MFMA of {h}: register v{r} holds the read of {read_of.get(ri)}"
                    assert (name, off) == (op(f"{sd}{'lo' if q < 4 else 'hi'}{kh}"), 4096 * b), (h, e, r)
            first_half = s == 0 and kh == 0
            assert (e[4] == "0") == first_half and (e[4] == "0" or e[4] == e[1])
        elif e[0] == "store":
            assert not any(set(_regs(e[3])) & p for p in pending), "store of pending LDS data"
    assert mf_k == nblk * len(halves)
    # the MFMA's B-operand format: e5m2 A rows (blgp 1) or e4m3
    for (opn, args) in KPROGS[cfg.name][0]:
        if opn == "v_mfma_f32_32x32x64_f8f6f4":
            assert ("blgp:1" in args[3]) == cfg.a_e5m2 and "cbsz" not in args[3]
    # ---- slot reuse
    epi_events = []
    for n, (a, b) in enumerate(spans):
        for i in range(a, b):
            if ev[i][0] in ("ds_write_b64", "ds_write_b128") or (ev[i][0] == "read" and i not in read_of):
                epi_events.append((i, slot_of[(n, S - 1)]))
    uses = sorted([(read_span[h][1], slot_of[(h[0], h[1])]) for h in halves] + epi_events)
    for st in stages:
        pos = issue_pos[st][0]
        slot = slot_of[st]
        prior = [i for i, sl in uses if sl == slot and i < pos]
        if prior:
            assert any(max(prior) < bi < pos for bi in barriers), f"DMA of {st} into slot {slot} races a reader"
        later = [i for i, sl in uses if sl == slot and pos < i < read_span[(st[0], st[1], 0)][0]]
        assert not later, f"slot {slot} read after the DMA of {st}"
    for n, (a, b) in enumerate(spans):
        first_w = next(i for i in range(a, b) if ev[i][0] in ("ds_write_b64", "ds_write_b128"))
        last_h = [h for h in halves if h[0] == n][-1]
        assert any(read_span[last_h][1] < bi < first_w for bi in barriers), f"tile {n}: staging races reads"
    # ---- stores per tile: the wgrad epilogue's whole lines, bounded by the tile's rows
    for n, (a, b) in enumerate(spans):
        g, row0, rows, n0 = tiles[n]
        st_ev = [ev[i] for i in range(a, b) if ev[i][0] == "store"]
        sw = (32 * cfg.bm * (wave & 1) * scm + 32 * cfg.bn * (wave >> 1)) * 2
        wn = wave >> 1
        want = []
        for i in range(cfg.bm):
            if cfg.joint:
                j0 = cfg.bn - 1 if wn == 0 else -1
                for row, _, _ in GEN.Gen.joint_stores(wn):
                    want.append((sw + (32 * i + row) * 2 * scm + 64 * j0, op("gb")))
            for blocks in (cfg.pairs_wn1 if wn else cfg.pairs):
                for row, _, _ in GEN.Gen.PAIR_STORES:
                    want.append((sw + (32 * i + row) * 2 * scm + 64 * blocks[0], op("gb")))
        assert sorted((e[1][0], e[1][1]) for e in st_ev) == sorted(want)
        for e in st_ev:
            base, nrec, _, _ = e[2]
            assert base == OUT + 2 * (row0 * scm + n0) and nrec == (rows * scm - n0) * 2
    assert state["np"] == 0 and state["nis"] == 0
    return ev


def _tiles(cfg, n, seed):
    rng = np.random.default_rng(seed)
    out, row = [], 0
    for _ in range(n):
        rows = int(rng.choice([1, 17, 255, 256, 256, 256]))
        out.append((int(rng.integers(0, 32)), row, rows, cfg.tn * int(rng.integers(0, 18))))
        row += rows
    return out


K_CASES = [64, 128, 192, 256, 2880, 5760, 448]


@pytest.mark.parametrize("cfg", list(KCFGS))
@pytest.mark.parametrize("K", K_CASES)
@pytest.mark.parametrize("ntiles", [1, 2, 3, 5])
def test_kmajor_pipeline_program(cfg, K, ntiles):
    c = KCFGS[cfg]
    _check(c, _tiles(c, ntiles, seed=K + ntiles), K)


@pytest.mark.parametrize("cfg", list(KCFGS))
@pytest.mark.parametrize("wave", [1, 2, 3])
def test_kmajor_other_waves(cfg, wave):
    c = KCFGS[cfg]
    _check(c, _tiles(c, 4, seed=wave), 2880, wave=wave)
    _check(c, _tiles(c, 3, seed=wave + 7), 512, wave=wave, sam=5760, sbn=5760, scm=2880)


@pytest.mark.parametrize("cfg", list(KCFGS))
def test_kmajor_waves_take_the_same_path(cfg):
    c = KCFGS[cfg]
    tiles = _tiles(c, 4, seed=3)
    seqs = []
    for wave in range(4):
        ev, _, _ = _run(c, tiles, 2880, wave, 2880, 5760 * 2880, 2880, 5760)
        seqs.append([e[0] for e in ev if e[0] in ("barrier", "mfma", "vmcnt", "lgkmcnt")])
    assert all(s == seqs[0] for s in seqs)


def test_kmajor_asm_writes_only_clobbered_registers():
    for c in GEN.KCONFIGS:
        g = GEN.GenK(c)
        g.tile()
        vset, sset = set(c.vgpr_clobber), set(c.sgpr_clobber)
        for line in g.lines:
            if line.endswith(":"):
                continue
            op, _, rest = line.partition(" ")
            if not rest or op.startswith(("s_cbranch", "s_branch", "s_waitcnt", "s_nop", "s_barrier",
                                          "buffer_store", "ds_write")) or "lds" in rest.split()[-1]:
                continue
            dst = rest.split(",")[0].strip()
            for m in re.finditer(r"\bv(\d+)\b|v\[(\d+):(\d+)\]", dst):
                lo, hi = (int(m.group(1)), int(m.group(1))) if m.group(1) else (int(m.group(2)), int(m.group(3)))
                assert set(range(lo, hi + 1)) <= vset, line
            for m in re.finditer(r"\bs(\d+)\b|s\[(\d+):(\d+)\]", dst):
                lo, hi = (int(m.group(1)), int(m.group(1))) if m.group(1) else (int(m.group(2)), int(m.group(3)))
                assert set(range(lo, hi + 1)) <= sset, line


def _swz(r):
    return (r & 7) ^ ((r >> 3) & 1)


def _dma_map(cfg, wave, j):
    """(row, logical chunk) lane l of LDS-DMA instruction j of `wave` writes, as persistent_wide.h
    sets its offsets, and the slot byte it lands at."""
    out = []
    for lane in range(64):
        lc = (lane & 7) ^ (lane >> 3) ^ (wave & 1)
        row = 8 * (wave + 4 * j) + (lane >> 3)
        if j >= cfg.nl:
            row = 8 * (wave + 4 * (j - cfg.nl)) + (lane >> 3)
        out.append((row, lc, 1024 * (wave + 4 * j) + 16 * lane))
    return out


@pytest.mark.parametrize("cfg", list(KCFGS))
def test_kmajor_dma_placement(cfg):
    """Every slot byte is written once per stage, at row r's physical chunk (logical ^ swz(r))."""
    c = KCFGS[cfg]
    seen = {}
    for wave in range(4):
        for j in range(c.loads):
            for row, lc, byte in _dma_map(c, wave, j):
                side_off = c.rhs_off if j >= c.nl else 0
                assert byte == side_off + row * 128 + 16 * (lc ^ _swz(row))
                assert byte not in seen
                seen[byte] = (j >= c.nl, row, lc)
    assert sorted(seen) == list(range(0, c.slot, 16))
    assert max(r for (b, r, _) in seen.values() if not b) == c.tm - 1
    assert max(r for (b, r, _) in seen.values() if b) == c.tn - 1


def _read_addr(cfg, side, wave, kh, x, b, lane):
    """Slot byte of lane `lane`'s read x (lo / hi) of block b, K-half kh (persistent_wide.h)."""
    wm, wn = wave & 1, wave >> 1
    rr, hh = lane & 31, lane >> 5
    row = (128 * wm if side == "am" else 160 * wn) + rr
    chunk = (4 * kh + 2 * hh + x) ^ _swz(rr)
    base = (0 if side == "am" else cfg.rhs_off) + row * 128 + 16 * chunk
    return base + 4096 * b


@pytest.mark.parametrize("cfg", list(KCFGS))
def test_kmajor_reads_match_dma_and_share_the_k_order(cfg):
    """Lane l's lo / hi reads of block b hold row 32 b + l % 32 (of the wave's rows), logical
    chunks 4 kh + 2 (l / 32) + (0, 1): the same K bytes for both operands (the MFMA pairs A lane l
    with B lane l' of the same l / 32), covering the 64 K bytes of the half once per row."""
    c = KCFGS[cfg]
    placed = {}
    for wave in range(4):
        for j in range(c.loads):
            for row, lc, byte in _dma_map(c, wave, j):
                placed[byte] = (j >= c.nl, row, lc)
    for wave in range(4):
        wm, wn = wave & 1, wave >> 1
        for kh in (0, 1):
            for side, nb in (("am", c.bm), ("bn", c.bn)):
                for b in range(nb):
                    cover = {}
                    for lane in range(64):
                        for x in (0, 1):
                            isb, row, lc = placed[_read_addr(c, side, wave, kh, x, b, lane)]
                            assert isb == (side == "bn")
                            want_row = (128 * wm if side == "am" else 160 * wn) + 32 * b + (lane & 31)
                            assert row == want_row and lc == 4 * kh + 2 * (lane >> 5) + x
                            cover.setdefault(row, set()).add(lc)
                    assert all(v == set(range(4 * kh, 4 * kh + 4)) for v in cover.values()) and len(cover) == 32


@pytest.mark.parametrize("cfg", list(KCFGS))
def test_kmajor_reads_conflict_free(cfg):
    """A 128-bit read is served 8 lanes at a time: each group of 8 lanes covers all 32 banks once."""
    c = KCFGS[cfg]
    for wave in range(4):
        for kh in (0, 1):
            for side, nb in (("am", c.bm), ("bn", c.bn)):
                for x in (0, 1):
                    for g in range(8):
                        banks = []
                        for lane in range(8 * g, 8 * g + 8):
                            a = _read_addr(c, side, wave, kh, x, 0, lane)
                            banks += [(a // 4 + k) % 32 for k in range(4)]
                        assert sorted(banks) == list(range(32))


def test_generated_include_lists_kmajor_configs():
    text = open(W.GEN_PATH.replace("gen_vark_wide.py", "vark_wide_asm.inc")).read()
    for c in GEN.KCONFIGS:
        assert f"#define GGEMM_WIDE_NOPERANDS_{c.name} {len(c.operands)}" in text


@pytest.mark.parametrize("cfg", [c.name for c in GEN.CONFIGS + GEN.KCONFIGS])
def test_only_mfma_writes_accumulators(cfg):
    """Accumulator registers (AGPRs and the VGPRs from vacc0 up) are written by MFMAs alone: no
    epilogue temporary, LDS load or address computation of any configuration lands on them. The
    one exception is by design: the fp32-accumulate epilogue loads old C values into the VGPRs of a
    block whose pass has already scaled them -- every v_mul_f32 reading such a register comes
    earlier in the (straight-line) epilogue than the load that overwrites it."""
    c = {x.name: x for x in GEN.CONFIGS + GEN.KCONFIGS}[cfg]
    g = GEN.GenK(c) if isinstance(c, GEN.KConfig) else GEN.Gen(c)
    g.tile()
    reused = 0
    for n, line in enumerate(g.lines):
        if line.endswith(":"):
            continue
        op, _, rest = line.partition(" ")
        if not rest or op.startswith(("v_mfma", "s_", "buffer_store", "ds_write")) or "lds" in rest.split()[-1]:
            continue
        dst = rest.split(",")[0].strip()
        assert not dst.startswith("a"), line
        for m in re.finditer(r"\bv(\d+)\b|v\[(\d+):(\d+)\]", dst):
            lo = int(m.group(1) or m.group(2))
            hi = int(m.group(1) or m.group(3))
            if hi < c.vacc0 or lo >= 256:
                continue
            assert c.out == "f32acc" and op == "buffer_load_dwordx4", line
            regs = {f"v{r}" for r in range(lo, hi + 1)}
            reads = [k for k, ln in enumerate(g.lines) if ln.startswith("v_mul_f32 ")
                     and ln.split(",")[-1].strip() in regs]
            assert reads and max(reads) < n, line
            reused += 1
    assert (reused > 0) == (c.out == "f32acc")
