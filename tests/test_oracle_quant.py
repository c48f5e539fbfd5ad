"""Pins the quantization oracle (oracle/quant_oracle.py) without trusting it.

Independent sources: torch's own float8 casts (every fp8 value, every tie between neighbours,
both fp32 neighbours of each tie, random fp32 values), the torch restatements of the recipes in
``ggemm_asm_amd.inputs`` (the generators of the measured configurations), exact rational
arithmetic for the MX exponent rule, and quantizing zero-padded groups one by one for the
padded layout.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

TDT = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _torch_cast(x: np.ndarray, fmt: str) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(TDT[fmt]).view(torch.uint8).numpy()


def _fp8_values(fmt):
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    v = b.view(TDT[fmt]).float().numpy()
    return np.sort(np.unique(v[np.isfinite(v) & (v >= 0)]))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_encoder_matches_torch_on_values_ties_and_neighbours(orq, fmt):
    vals = _fp8_values(fmt)
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)   # exact ties
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(0))
    rng = np.random.default_rng(0)
    fmax = float(orq.FMAX[fmt])
    rnd = (rng.uniform(-1, 1, 200000) * np.float32(2.0) ** rng.integers(-40, 17, 200000)).astype(np.float32)
    rnd = rnd[np.abs(rnd) <= fmax]
    tiny = (np.arange(1, 5000, dtype=np.uint32)).view(np.float32)                  # fp32 subnormals
    x = np.concatenate([vals, mids, up, dn, rnd, tiny, [0.0, fmax]]).astype(np.float32)
    x = x[np.abs(x) <= fmax]
    x = np.concatenate([x, -x, np.array([-0.0], np.float32)])
    np.testing.assert_array_equal(orq.encode_fp8(x, fmt), _torch_cast(x, fmt))
    # ties round to the even neighbour: every tie's code is even in its low mantissa bit
    assert np.all(orq.encode_fp8(mids, fmt) % 2 == 0)
    assert orq.encode_fp8(np.array([np.nan], np.float32), fmt)[0] == 0x7F


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_tensorwise_matches_torch_recipe(pkg, orq, fmt, dtype):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn((257, 96), generator=g) * (1e-3 if fmt == "e5m2" else 1.0)).to(dtype)
    q_ref, s_ref = pkg.inputs.quantize_tensorwise(x.float(), fmt)
    q, scale, am = orq.quantize_tensorwise(x.float().numpy(), fmt)
    assert np.float32(scale) == np.float32(s_ref)
    assert am == np.float32(x.float().abs().max())
    np.testing.assert_array_equal(q, q_ref.numpy())
    # the scale divides amax by fmax exactly as fp32 division does
    assert scale == np.float32(np.float32(am) / orq.FMAX[fmt])


def test_tensorwise_special_cases(orq):
    q, scale, am = orq.quantize_tensorwise(np.zeros((4, 8), np.float32), "e4m3")
    assert scale == 1.0 and am == 0.0 and np.all(q == 0)
    x = np.zeros((2, 8), np.float32)
    x[0, 3] = np.nan
    q, scale, am = orq.quantize_tensorwise(x, "e5m2")
    assert np.isnan(am) and np.isnan(scale) and np.all((q & 0x7F) == 0x7F)
    # amax maps to fmax exactly; values keep their sign
    x = np.array([[-3.0, 1.5, 0.0, -0.0, 3.0, 0.75, -1.5, 0.375]], np.float32)
    q, scale, _ = orq.quantize_tensorwise(x, "e4m3")
    assert q[0, 4] == 0x7E and q[0, 0] == 0xFE and q[0, 3] == 0x80 and q[0, 2] == 0


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_mx_exponent_rule_exact(orq, fmt):
    """X = floor(log2(fl32(amax / fmax))) checked with exact rationals at, just below and just
    above powers of two of the quotient, and on random amax values."""
    fmax = Fraction(int(orq.FMAX[fmt]))
    ys = []
    for k in range(-126, 127, 7):
        p = np.float32(2.0) ** k
        ys += [p, np.nextafter(p, np.float32(0)), np.nextafter(p, np.float32(np.inf))]
    rng = np.random.default_rng(1)
    ys += list((rng.uniform(0.5, 1, 2000) * np.float32(2.0) ** rng.integers(-120, 120, 2000)).astype(np.float32))
    with np.errstate(over="ignore"):
        am = np.array([np.float32(y) * orq.FMAX[fmt] for y in ys], np.float32)
    am = am[np.isfinite(am) & (am > 0)]
    X = orq.block_exponent(am, fmt)
    for a, x in zip(am, X):
        y = Fraction(float(np.float32(np.float32(a) / orq.FMAX[fmt])))   # the fp32 quotient, exactly
        e = y.numerator.bit_length() - y.denominator.bit_length()
        if Fraction(2) ** e > y:
            e -= 1
        assert Fraction(2) ** e <= y < Fraction(2) ** (e + 1)
        assert x == max(-127, min(127, e)), (a, x, e)
    assert orq.block_exponent(np.array([0.0, np.nan, np.inf], np.float32), fmt).tolist() == [0, 128, 127]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_mx_matches_torch_recipe_on_aligned_groups(pkg, orq, fmt):
    g = torch.Generator().manual_seed(4)
    x = torch.randn((256, 80), generator=g) * (1e-3 if fmt == "e5m2" else 1.0)
    x[64:96] = 0                                                          # an all-zero block
    x[100, 7] = 1e-30                                                     # tiny block maxima
    q_ref, s_ref = pkg.inputs.quantize_mx(x, fmt)
    offs = np.array([0, 64, 64, 160, 256], np.int64)                      # starts already 32-aligned
    q, sc, pad = orq.quantize_mx_grouped(x.numpy(), offs, fmt, out_rows=256)
    np.testing.assert_array_equal(pad, offs)
    np.testing.assert_array_equal(sc, s_ref.numpy())
    np.testing.assert_array_equal(q, q_ref.numpy())


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_mx_padding_equals_per_group_padded_quantization(pkg, orq, fmt):
    lens = [5, 0, 33, 64, 1, 100]
    g = torch.Generator().manual_seed(5)
    M = sum(lens)
    x = torch.randn((M, 48), generator=g)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    q, sc, pad = orq.quantize_mx_grouped(x.numpy(), offs, fmt)
    assert q.shape[0] == (M + 31 * len(lens) + 31) // 32 * 32
    np.testing.assert_array_equal(pad, np.concatenate([[0], np.cumsum([(l + 31) // 32 * 32 for l in lens])]))
    for gi, L in enumerate(lens):
        P = (L + 31) // 32 * 32
        if P == 0:
            continue
        xg = torch.zeros((P, 48))
        xg[:L] = x[offs[gi]:offs[gi + 1]]
        q_ref, s_ref = pkg.inputs.quantize_mx(xg, fmt)
        np.testing.assert_array_equal(q[pad[gi]:pad[gi] + P], q_ref.numpy())
        np.testing.assert_array_equal(sc[pad[gi] // 32:pad[gi] // 32 + P // 32], s_ref.numpy())
    assert np.all(q[pad[-1]:] == 0)


def test_mx_dequantized_error_bound(orq):
    """Dequantized MX values are within half an e4m3 ulp of x (|err| <= 2^-4 |x| in the normal
    range, <= 2^-10 * 2^X below it) unless x / 2^X exceeds 448 and saturates to +-448 * 2^X."""
    rng = np.random.default_rng(6)
    x = rng.standard_normal((128, 64)).astype(np.float32)
    q, sc, pad = orq.quantize_mx_grouped(x, np.array([0, 128]), "e4m3", out_rows=128)
    scale = np.ldexp(np.float32(1.0), sc.astype(np.int32) - 127).repeat(32, axis=0)
    deq = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy() * scale
    y = x / scale
    sat = np.abs(y) > 448
    assert np.all(deq[sat] == np.sign(x[sat]) * 448 * scale[sat])
    err = np.abs(deq - x)[~sat]
    assert np.all(err <= np.maximum(np.abs(x[~sat]) * 2.0 ** -4, 2.0 ** -10 * scale[~sat]))
    assert sat.any()          # the recipe puts block maxima in [448, 896): some saturate


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_delayed_matches_torch_recipe(orq, fmt):
    """The delayed recipe against torch: scale = max(|history| without the slot) / fmax by torch's
    own max and fp32 division, bytes by torch's float8 cast of clamp(x / scale); the slot's old
    entry (here the largest) plays no part; the new history differs from the old one at the slot
    only, where it holds max |x|."""
    rng = np.random.default_rng(11)
    fmax = float(orq.FMAX[fmt])
    x = (rng.standard_normal((300, 64)) * (1e-3 if fmt == "e5m2" else 1.0)).astype(np.float32)
    am = float(np.abs(x).max())
    for hist_scale in (0.5, 1.0, 2.0):                       # values past the history's range saturate
        hist = (rng.uniform(0.2, 1.0, 16) * am * hist_scale).astype(np.float32)
        slot = 5
        hist[slot] = 1e9
        q, scale, h2 = orq.quantize_tensorwise_delayed(x, hist, slot, fmt)
        ht = torch.from_numpy(hist)
        m = torch.cat([ht[:slot], ht[slot + 1:]]).abs().max()
        s_ref = m / torch.tensor(fmax, dtype=torch.float32)
        assert np.float32(scale) == np.float32(s_ref.item())
        y = torch.clamp(torch.from_numpy(x) / s_ref, -fmax, fmax)
        np.testing.assert_array_equal(q, y.to(TDT[fmt]).view(torch.uint8).numpy())
        assert h2[slot] == np.float32(am)
        np.testing.assert_array_equal(np.delete(h2, slot), np.delete(hist, slot))
        n_sat = int(np.sum(np.abs(x) / np.float32(scale) > fmax))
        sat = 0x7E if fmt == "e4m3" else 0x7B
        assert int(np.sum((q & 0x7F) == sat)) >= n_sat and (hist_scale >= 1.0 or n_sat > 0)


def test_delayed_special_histories(orq):
    x = np.array([[1.0, -2.0, 0.0, 1e6, -1e6, 0.5, 3.0, -0.0]], np.float32)
    # all other entries zero: scale 1, x / 1 clamped (1e6 saturates)
    q, scale, h2 = orq.quantize_tensorwise_delayed(x, np.array([0.0, 7.0, 0.0], np.float32), 1, "e4m3")
    assert scale == 1.0 and h2[1] == np.float32(1e6)
    np.testing.assert_array_equal(q, orq.encode_fp8(np.clip(x, -448, 448), "e4m3"))
    assert q[0, 3] == 0x7E and q[0, 4] == 0xFE
    # a NaN entry: NaN scale and NaN codes; a NaN in x reaches the new entry
    q, scale, _ = orq.quantize_tensorwise_delayed(x, np.array([np.nan, 1.0], np.float32), 1, "e5m2")
    assert np.isnan(scale) and np.all((q & 0x7F) == 0x7F)
    y = x.copy()
    y[0, 2] = np.nan
    _, _, h2 = orq.quantize_tensorwise_delayed(y, np.array([1.0, 1.0], np.float32), 0, "e5m2")
    assert np.isnan(h2[0]) and h2[1] == 1.0
    # a one-entry history has no other entries: scale 1
    _, scale, _ = orq.quantize_tensorwise_delayed(x, np.array([5.0], np.float32), 0, "e4m3")
    assert scale == 1.0
    # the largest entry by magnitude, sign ignored (histories hold amax values; a negative entry
    # is read as its magnitude, as the device reads the bits without the sign)
    _, scale, _ = orq.quantize_tensorwise_delayed(x, np.array([-896.0, 448.0, 0.0], np.float32), 2, "e4m3")
    assert scale == 2.0
