"""CPU model of the variable-K kernel's persistent schedule (make_sched in
ggemm-asm_amd/csrc/vark_kernel.h; no kernel launches).

The kernel deals the size-sorted tile list to its workgroups in one of two static deals (equal-work
slices per XCD pair, or boustrophedon rounds over all workgroups) and takes the one whose heaviest
workgroup is lighter. The model restates that integer arithmetic and checks: every deal covers each
tile exactly once for any grid; the choice is the lighter deal; skewed routing (the reference's
exponential lengths, Zipf) takes the rounds deal, uniform routing keeps the slices; and the chosen
deal's heaviest workgroup is within a few percent of the average on the measured shapes.
"""
import numpy as np
import pytest
import torch

TILE_M, K_STEP, XCDS, PAIRS = 192, 128, 8, 4


def _tn(OUT_N):
    """wide_tiles() of the per-tensor kernel: 384 for multiples of 384, and when at least four
    tiles fit and the last is at least half full."""
    return 384 if OUT_N % 384 == 0 or (OUT_N >= 4 * 384 and OUT_N % 384 >= 192) else 320


def _schedule(lens, OUT_M, OUT_N, num_wg, epi_w=1):
    """(tiles per group, sorted order, weights per sorted slot, {deal: [tile list per workgroup]},
    chosen deal)."""
    G = len(lens)
    order = sorted(range(G), key=lambda g: (-max(lens[g], 0), g))          # stable descending rank
    tpg = -(-OUT_M // TILE_M) * -(-OUT_N // _tn(OUT_N))
    total = G * tpg
    w_slot = [(-(-max(lens[g], 0) // K_STEP)) + epi_w for g in order]
    spread = num_wg % XCDS == 0
    xcds = XCDS if spread else 1
    n_x = PAIRS if spread else 1
    per_slice, wpx = xcds // n_x, num_wg // xcds
    if n_x > 1:
        total_w = sum(tpg * w for w in w_slot)
        bounds, acc, x = [0], 0, 1
        for sl, w in enumerate(w_slot):
            if x >= n_x:
                break
            while x < n_x and acc + w * tpg >= total_w * x // n_x:
                need = total_w * x // n_x - acc
                i = -(-need // w)
                bounds.append(sl * tpg + min(i, tpg))
                x += 1
            acc += w * tpg
        bounds += [total] * (n_x + 1 - len(bounds))
    else:
        bounds = [total * x // n_x for x in range(n_x + 1)]

    def walk(first, end, d0, d1):
        out, t, d, da = [], first, d0, d1
        while t < end:
            out.append(t)
            t, d, da = t + d, da, d
        return out

    def slices(w):
        xcd = w % xcds
        sl, part = xcd % n_x, xcd // n_x
        step = per_slice * wpx
        return walk(bounds[sl] + part * wpx + w // xcds, bounds[sl + 1], step, step)

    def rounds(w):
        p = (w % xcds) * wpx + w // xcds
        return walk(p, total, 2 * (num_wg - p) - 1, 2 * p + 1)

    deals = {"slices": [slices(w) for w in range(num_wg)], "rounds": [rounds(w) for w in range(num_wg)]}
    heaviest = {k: max(sum(w_slot[t // tpg] for t in ts) for ts in v) for k, v in deals.items()}
    chosen = "rounds" if n_x > 1 and heaviest["rounds"] < heaviest["slices"] else "slices"
    return tpg, order, w_slot, deals, chosen, heaviest


def _load_ratio(lens, num_wg=256, epi_w=1, OUT_M=2880, OUT_N=5760):
    tpg, _, w_slot, deals, chosen, heaviest = _schedule(lens, OUT_M, OUT_N, num_wg, epi_w)
    avg = sum(tpg * w for w in w_slot) / num_wg
    return chosen, heaviest[chosen] / avg, heaviest


@pytest.mark.parametrize("lens,OUT_M,OUT_N,grids", [
    ([96, 160, 0, 256], 64, 128, (256, 1, 8, 24)),
    ([1000, 0, 7, 4096, 193, 192, 0], 2880, 5760, (256, 20, 8, 304)),
    ([5, 3], 2880, 2880, (256, 1, 16)),
    ([4000] * 32, 2880, 2880, (256, 64)),
])
def test_both_deals_cover_every_tile_once(lens, OUT_M, OUT_N, grids):
    for num_wg in grids:
        tpg, _, _, deals, _, _ = _schedule(lens, OUT_M, OUT_N, num_wg)
        for name, per_wg in deals.items():
            seen = sorted(t for ts in per_wg for t in ts)
            assert seen == list(range(len(lens) * tpg)), (name, num_wg)
            for ts in per_wg:
                assert all(a < b for a, b in zip(ts, ts[1:])), (name, num_wg)   # increasing: the loop's exit test


def test_rounds_deal_keeps_xcd_blocks_of_32():
    """In every round, the 32 workgroups of one XCD (ids x, x + 8, ...) hold 32 consecutive tiles."""
    _, _, _, deals, _, _ = _schedule([4096] * 32, 2880, 5760, 256)
    per_wg = deals["rounds"]
    for r in range(len(per_wg[0])):
        for x in range(XCDS):
            ts = sorted(per_wg[w][r] for w in range(x, 256, XCDS) if r < len(per_wg[w]))
            if len(ts) == 32:
                assert ts == list(range(ts[0], ts[0] + 32))


def test_choice_follows_routing(pkg):
    """Skewed routing (the reference's seed-42 exponential lengths; Zipf(1.2) with empty and tiny
    groups) takes the rounds deal, uniform multinomial routing the slices; the chosen deal's
    heaviest workgroup stays within 5% of the average weight (7% for the Zipf lengths, whose largest
    group holds a third of the tokens)."""
    ref = [int(v) for v in pkg.inputs.make_group_lens_reference()]
    zipf = [int(v) for v in pkg.inputs.zipf_lens(32, 131072, torch.Generator().manual_seed(0), n_empty=4, n_tiny=8)]
    multi = [int(v) for v in pkg.inputs.multinomial_lens(32, 131072, torch.Generator().manual_seed(0))]
    for lens, want in [(ref, "rounds"), (zipf, "rounds"), (multi, "slices")]:
        for epi_w in (1, 2, 4):
            chosen, ratio, heaviest = _load_ratio(lens, epi_w=epi_w)
            assert chosen == want, (want, epi_w, heaviest)
            assert ratio < (1.07 if lens is zipf else 1.05), (want, epi_w, ratio)
    # with the reference lengths the slice deal's heaviest workgroup carries 9% more than the
    # rounds deal's (the slice holding the largest groups ends late)
    _, _, heaviest = _load_ratio(ref)
    assert heaviest["slices"] > 1.08 * heaviest["rounds"]


def test_unspread_grid_keeps_slices():
    """A grid that is not a multiple of the XCD count has one slice and no choice."""
    _, _, _, _, chosen, _ = _schedule([18000, 10, 10, 10], 2880, 5760, 20)
    assert chosen == "slices"


def _tile_in_group(in_g, n_tm, n_tn, band_n=4):
    """tile_at's walk inside a group (vark_kernel.h): bands of band_n N-tiles, M-tile by M-tile
    inside a band, down the M-tiles in even bands and back up in odd ones."""
    band = in_g // (n_tm * band_n)
    r = in_g - band * n_tm * band_n
    bw = min(band_n, n_tn - band * band_n)
    tr = r // bw
    tm = n_tm - 1 - tr if band & 1 else tr
    return tm, band * band_n + (r - tr * bw)


def test_tile_walk_matches_kernel_and_covers_each_tile_once():
    import os
    import re
    from conftest import ROOT
    text = open(os.path.join(ROOT, "ggemm-asm_amd", "csrc", "vark_kernel.h")).read()
    assert re.findall(r"constexpr int kBandN = (\d+);", text) == ["4"]
    assert text.count("const int tm = (band & 1) ? S.n_tm - 1 - tr : tr;") == 1
    for n_tm, n_tn in [(9, 18), (15, 15), (9, 9), (1, 1), (3, 7), (16, 5), (2, 13)]:
        seen = [_tile_in_group(i, n_tm, n_tn) for i in range(n_tm * n_tn)]
        assert sorted(seen) == [(a, b) for a in range(n_tm) for b in range(n_tn)], (n_tm, n_tn)


def test_serpentine_rounds_share_panels():
    """Where 32 consecutive tiles of a group cross from one band into the next, the serpentine
    walk keeps them on the M-tiles the band just ended on: at gate_up's 9 x 18 grid of 320 x 320
    tiles, the distinct LHS + RHS panels summed over every 32-tile window are fewer than with every
    band walked downward (the panel count is what an XCD's L2 fetches per token of the group)."""
    n_tm, n_tn = 9, 18

    def panels(walk):
        tot = 0
        for s in range(0, n_tm * n_tn - 31):
            w = [walk(i) for i in range(s, s + 32)]
            tot += len({a for a, _ in w}) + len({b for _, b in w})
        return tot

    def one_way(i):
        band, r = divmod(i, n_tm * 4)
        bw = min(4, n_tn - band * 4)
        return r // bw, band * 4 + r % bw

    assert panels(lambda i: _tile_in_group(i, n_tm, n_tn)) < 0.95 * panels(one_way)
