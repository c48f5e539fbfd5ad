"""Pins the CPU oracle (oracle/vark_oracle.py, oracle/vark_oracle.c) without trusting it.

The reference holds no golden vectors for this path (its only check is a live cosine >= 0.999
against a Triton kernel that is not available here), so each oracle function is pinned by an
independent source: torch's own fp8/bf16 codecs, exact rational brute force, closed forms
(launcher.cpp's constant fill), algebraic invariants, and the reference generator's recorded
seed-42 output.
"""
import ctypes
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from conftest import GOLDEN, ROOT


# ----------------------------------------------------------------------------- codecs

def test_e4m3_table_matches_torch(orc):
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = b.view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(orc.E4M3_TABLE), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(orc.E4M3_TABLE[ok], ref[ok])


def test_e5m2_table_matches_torch(orc):
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = b.view(torch.float8_e5m2).float().numpy()
    np.testing.assert_array_equal(np.isnan(orc.E5M2_TABLE), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(orc.E5M2_TABLE[ok], ref[ok])


def test_fp8_textbook_values(orc):
    # launcher.cpp:106 fills 0x38: 1.0 as e4m3fn, 0.5 as e5m2
    assert orc.E4M3_TABLE[0x38] == 1.0 and orc.E5M2_TABLE[0x38] == 0.5
    assert orc.E4M3_TABLE[0x7E] == 448.0 and orc.E4M3_TABLE[0xFE] == -448.0
    assert np.isnan(orc.E4M3_TABLE[0x7F]) and np.isnan(orc.E4M3_TABLE[0xFF])
    assert orc.E5M2_TABLE[0x7B] == 57344.0 and np.isinf(orc.E5M2_TABLE[0x7C])
    assert orc.E4M3_TABLE[0x01] == 2.0 ** -9 and orc.E5M2_TABLE[0x01] == 2.0 ** -16
    assert orc.E4M3_TABLE[0x80] == 0.0 and np.signbit(orc.E4M3_TABLE[0x80])


def test_e8m0_decode(orc):
    b = np.array([0, 1, 126, 127, 128, 254, 255], dtype=np.uint8)
    d = orc.decode_e8m0(b)
    assert d[3] == 1.0 and d[2] == 0.5 and d[4] == 2.0 and d[5] == 2.0 ** 127
    assert d[1] == 2.0 ** -126 and d[0] == 2.0 ** -127 and np.isnan(d[6])
    if hasattr(torch, "float8_e8m0fnu"):
        t = torch.tensor(b[:-1]).view(torch.float8_e8m0fnu).float().numpy()
        np.testing.assert_array_equal(d[:-1], t)


def test_bf16_rne_matches_torch(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0, 1.00390625, 1.01171875, 3.3895314e38, 1e-40, -1e-42],
                 dtype=np.float32),
        # exact ties: low 16 bits 0x8000 with even and odd kept bit
        (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x00008000, 0x7F7F8000], dtype=np.uint32)).view(np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.bf16_bits_rne(x)
    np.testing.assert_array_equal(got, ref)
    assert orc.bf16_bits_rne(np.array([np.nan], dtype=np.float32))[0] == 0x7FC0


# ----------------------------------------------------------------------------- GEMM vs exact

def _rand_problem(rng, lens, om, on, nan_free=True):
    M = int(sum(lens))
    lhs = rng.integers(0, 256, (M, om), dtype=np.uint8)
    rhs = rng.integers(0, 256, (M, on), dtype=np.uint8)
    if nan_free:  # keep to finite codes: e4m3 0x7F/0xFF NaN, e5m2 exponent 31 inf/NaN
        lhs[(lhs & 0x7F) == 0x7F] = 0x3A
        rhs[(rhs & 0x7C) == 0x7C] = 0x3B
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    return lhs, rhs, offs


@pytest.mark.parametrize("lens", [[1, 0, 3], [31, 2, 0, 5], [7], [0, 0, 9], [17, 13]])
def test_oracle_vs_exact_bruteforce(orc, lens):
    """fp32 oracle within the textbook error bound of the exact rational result:
    |fp32 - exact| <= (K + 2) * 2^-24 * sum_k |terms| (two dequantize roundings per term plus
    K-term fp32 summation), and exactly zero for empty groups."""
    rng = np.random.default_rng(len(lens) * 100 + sum(lens))
    lhs, rhs, offs = _rand_problem(rng, lens, 5, 7)
    sl, sr = 0.0123, 3.7e-5
    exact, mag = orc.vark_wgrad_bruteforce_exact(lhs, rhs, sl, sr, offs)
    f32 = orc.vark_wgrad_tensorwise_f32(lhs, rhs, sl, sr, offs)
    for g, K in enumerate(lens):
        for m in range(5):
            for n in range(7):
                err = abs(Fraction(float(f32[g, m, n])) - exact[g][m][n])
                assert err <= Fraction(K + 2, 2 ** 24) * mag[g][m][n] + Fraction(1, 2 ** 140)
                if K == 0:
                    assert f32[g, m, n] == 0
    # power-of-two scales make the dequantize exact; float64 contraction of <= 31 terms whose
    # exponents span < 2^45 is then exact as well
    exact1, _ = orc.vark_wgrad_bruteforce_exact(lhs, rhs, 0.5, 0.25, offs)
    f64 = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 0.5, 0.25, offs, acc_dtype=np.float64)
    mism = sum(Fraction(float(f64[g, m, n])) != exact1[g][m][n]
               for g in range(len(lens)) for m in range(5) for n in range(7))
    assert mism == 0


def test_empty_groups_exact_zero(orc):
    rng = np.random.default_rng(1)
    lhs, rhs, offs = _rand_problem(rng, [0, 4, 0, 0, 6, 0], 16, 32)
    bits = orc.vark_wgrad_tensorwise(lhs, rhs, 0.5, 0.25, offs)
    for g in (0, 2, 3, 5):
        assert np.all(bits[g] == 0)


def test_single_group_is_plain_matmul(orc):
    rng = np.random.default_rng(2)
    lhs, rhs, offs = _rand_problem(rng, [300], 48, 40)
    a = orc.E4M3_TABLE[lhs].astype(np.float64) * np.float64(np.float32(0.01))
    b = orc.E5M2_TABLE[rhs].astype(np.float64) * np.float64(np.float32(2.5e-3))
    ref = np.einsum("km,kn->mn", a, b)
    got = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 0.01, 2.5e-3, offs)[0]
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=1e-6 * np.abs(ref).max())


def test_constant_fill_closed_form(orc):
    """launcher.cpp:97-112 inputs: bytes 0x38, scales 0.1, K_g = 4096 -> C = 0.1*0.1*1.0*0.5*4096
    = 20.48 -> bf16 20.5 (0x41A4) everywhere."""
    K, om, on = 4096, 16, 32
    lhs = np.full((2 * K, om), 0x38, dtype=np.uint8)
    rhs = np.full((2 * K, on), 0x38, dtype=np.uint8)
    offs = np.array([0, K, 2 * K], dtype=np.int64)
    bits = orc.vark_wgrad_tensorwise(lhs, rhs, 0.1, 0.1, offs)
    assert np.all(bits == 0x41A4)
    assert orc.bf16_bits_to_f32(np.array([0x41A4], dtype=np.uint16))[0] == 20.5


def test_invariants_permutation_split_linearity(orc):
    rng = np.random.default_rng(3)
    lhs, rhs, offs = _rand_problem(rng, [50, 70], 24, 40)
    base = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 0.5, 0.125, offs, acc_dtype=np.float64)
    # token permutation inside group 1 leaves C unchanged
    perm = np.concatenate([np.arange(50), 50 + rng.permutation(70)])
    p = orc.vark_wgrad_tensorwise_f32(lhs[perm], rhs[perm], 0.5, 0.125, offs, acc_dtype=np.float64)
    np.testing.assert_allclose(p, base, rtol=1e-12, atol=1e-12)
    # splitting group 1 into 30 + 40 tokens: the halves sum to the whole
    s = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 0.5, 0.125, np.array([0, 50, 80, 120]), acc_dtype=np.float64)
    np.testing.assert_allclose(s[1] + s[2], base[1], rtol=1e-12, atol=1e-12)
    # a power-of-two scale is exactly linear
    l2 = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 1.0, 0.125, offs)
    l1 = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 0.5, 0.125, offs)
    np.testing.assert_array_equal(l2, 2 * l1)
    # appending zero-byte rows to a group changes nothing
    z = np.zeros((10, 24), np.uint8), np.zeros((10, 40), np.uint8)
    lz = np.concatenate([lhs, z[0]]); rz = np.concatenate([rhs, z[1]])
    e = orc.vark_wgrad_tensorwise_f32(lz, rz, 0.5, 0.125, np.array([0, 50, 130]), acc_dtype=np.float64)
    np.testing.assert_array_equal(e, base)


def test_mx_oracle_reduces_to_tensorwise_and_is_blockwise_linear(orc):
    rng = np.random.default_rng(4)
    lhs, rhs, offs = _rand_problem(rng, [64, 0, 96], 16, 32)
    nb = lhs.shape[0] // 32
    ones_l = np.full((nb, 16), 127, np.uint8)
    ones_r = np.full((nb, 32), 127, np.uint8)
    mx = orc.vark_wgrad_mxfp8_f32(lhs, rhs, ones_l, ones_r, offs, acc_dtype=np.float64)
    tw = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 1.0, 1.0, offs, acc_dtype=np.float64)
    np.testing.assert_array_equal(mx, tw)
    # bumping the LHS scale of token block 3 (group 2's second block) by +1 doubles that block
    sl = ones_l.copy(); sl[3, :] = 128
    bumped = orc.vark_wgrad_mxfp8_f32(lhs, rhs, sl, ones_r, offs, acc_dtype=np.float64)
    blk = orc.vark_wgrad_tensorwise_f32(lhs, rhs, 1.0, 1.0, np.array([0, 96, 128]), acc_dtype=np.float64)[1]
    np.testing.assert_allclose(bumped[2], tw[2] + blk, rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError):
        orc.vark_wgrad_mxfp8_f32(lhs, rhs, ones_l, ones_r, np.array([0, 40, 40, 160]))


# ----------------------------------------------------------------------------- C restatement

def _c_oracle():
    # GGEMM_ORACLE_C_LIBRARY: a variant build of vark_oracle.c (the host-sanitizer run)
    path = os.environ.get("GGEMM_ORACLE_C_LIBRARY") or os.path.join(ROOT, "oracle", "_build", "libvark_oracle_c.so")
    if not os.path.exists(path):
        from oracle import build
        build.build_c()
    lib = ctypes.CDLL(path)
    lib.vo_e4m3_to_f32.restype = ctypes.c_float
    lib.vo_e4m3_to_f32.argtypes = [ctypes.c_uint8]
    lib.vo_e5m2_to_f32.restype = ctypes.c_float
    lib.vo_e5m2_to_f32.argtypes = [ctypes.c_uint8]
    lib.vo_vark_tensorwise.restype = ctypes.c_int
    lib.vo_vark_tensorwise.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float,
                                       ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    lib.vo_persistent_fp8.restype = ctypes.c_int
    lib.vo_persistent_fp8.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_void_p,
                                      ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                      ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64]
    return lib


def test_c_oracle_decoders_match_tables(orc):
    lib = _c_oracle()
    for b in range(256):
        for fn, tab in ((lib.vo_e4m3_to_f32, orc.E4M3_TABLE), (lib.vo_e5m2_to_f32, orc.E5M2_TABLE)):
            v = fn(b)
            assert (np.isnan(v) and np.isnan(tab[b])) or v == tab[b]


def test_c_oracle_agrees_with_numpy_oracle(orc):
    lib = _c_oracle()
    rng = np.random.default_rng(5)
    lens = [33, 0, 129, 1, 200]
    lhs, rhs, offs = _rand_problem(rng, lens, 32, 48)
    out = np.zeros((len(lens), 32, 48), np.uint16)
    rc = lib.vo_vark_tensorwise(lhs.ctypes.data, rhs.ctypes.data, ctypes.c_float(0.02), ctypes.c_float(1e-4),
                                offs.ctypes.data, len(lens), lhs.shape[0], 32, 48, 32, 48, out.ctypes.data)
    assert rc == 0
    ref = orc.vark_wgrad_tensorwise(lhs, rhs, 0.02, 1e-4, offs)
    m = orc.compare(out, ref, offs)
    assert m["cos"] > 0.9999999 and m["max_rel"] <= 2 ** -7 and m["empty_zero"], m


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_c_persistent_oracle_agrees_with_numpy_oracle(orp, orc, fmt):
    """The C restatement of the persistent GEMM (vo_persistent_fp8) against the numpy one: ragged
    and empty groups, K not a multiple of 128, B rows strided past K, untouched rows outside every
    group (the sentinel 0x1234 stays)."""
    lib = _c_oracle()
    rng = np.random.default_rng(7 if fmt == "e4m3" else 8)
    lens, K, N = [37, 0, 130, 5], 208, 48
    M = sum(lens) + 3
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    dt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    a = torch.randn((M, K), generator=torch.Generator().manual_seed(1)).to(dt).view(torch.uint8).numpy()
    b_full = torch.randn((len(lens), N, K + 32), generator=torch.Generator().manual_seed(2)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    out = np.full((M, N), 0x1234, np.uint16)
    rc = lib.vo_persistent_fp8(a.ctypes.data, b_full.ctypes.data, ctypes.c_float(0.1), ctypes.c_float(0.05),
                               offs.ctypes.data, len(lens), M, N, K, K, N * (K + 32), K + 32, int(fmt == "e5m2"),
                               out.ctypes.data, N)
    assert rc == 0
    ref = orp.grouped_fp8(a, np.ascontiguousarray(b_full[:, :, :K]), 0.1, 0.05, offs, fmt)
    rows = int(offs[-1])
    m = orc.compare(out[:rows], ref[:rows])
    assert m["cos"] > 0.9999999 and m["max_rel"] <= 2 ** -7, m
    assert np.all(out[rows:] == 0x1234)
    bad = offs.copy()
    bad[2] = bad[1] - 1
    assert lib.vo_persistent_fp8(a.ctypes.data, b_full.ctypes.data, ctypes.c_float(1), ctypes.c_float(1),
                                 bad.ctypes.data, len(lens), M, N, K, K, N * (K + 32), K + 32, 0, out.ctypes.data,
                                 N) == -1


# ----------------------------------------------------------------------------- reference generator

RECORDED_SEED42_LENS = [350, 380, 772, 316, 4372, 3791, 18183, 15463, 510, 832, 1000, 2754, 10820, 11965,
                      2775, 5548, 539, 7070, 5716, 3365, 454, 6733, 2191, 2164, 186, 241, 15728, 966, 1802,
                      818, 1698, 1570]


def test_reference_group_lens_seed42(pkg):
    """reference bench.py:205-212 restated: the recorded seed-42 CPU lengths."""
    lens = pkg.inputs.make_group_lens_reference(32, 131072, 42)
    assert lens.tolist() == RECORDED_SEED42_LENS
    offs = pkg.inputs.make_group_offs(lens)
    assert offs[0] == 0 and offs[-1] == 131072 and offs.dtype == torch.int64


def test_wgrad_site_reference_recipe(pkg):
    """reference bench.py:221-223,731-737: randn bf16 cast straight to e4m3fn / e5m2, scales 0.1,
    the seed-42 lengths unless overridden."""
    p = pkg.inputs.make_wgrad_site_problem("down_wgrad", seed=5, lens=[40, 0, 24])
    assert (p.G, p.M, p.OUT_M, p.OUT_N) == (3, 64, 2880, 2880)
    assert p.lhs_scale == p.rhs_scale == 0.1 and p.group_offs.tolist() == [0, 40, 40, 64]
    gen = torch.Generator().manual_seed(5)
    ref_l = torch.randn((64, 2880), generator=gen, dtype=torch.bfloat16).to(torch.float8_e4m3fn)
    ref_r = torch.randn((64, 2880), generator=gen, dtype=torch.bfloat16).to(torch.float8_e5m2)
    assert torch.equal(p.lhs, ref_l.view(torch.uint8)) and torch.equal(p.rhs, ref_r.view(torch.uint8))
    assert pkg.inputs.make_wgrad_site_problem.__defaults__[0] == 42
    with pytest.raises(ValueError):
        pkg.inputs.make_wgrad_site_problem("gate_up_fwd")


def test_config_length_recipes(pkg):
    g = torch.Generator().manual_seed(0)
    z = pkg.inputs.zipf_lens(32, 131072, g)
    assert int(z.sum()) == 131072 and int((z == 0).sum()) >= 4
    assert int(((z >= 1) & (z <= 31)).sum()) >= 8 and int(z.max()) > 30000
    g = torch.Generator().manual_seed(0)
    mx = pkg.inputs.mx_lens(32, 131072, g)
    assert int(mx.sum()) == 131072 and bool((mx % 32 == 0).all())
    g = torch.Generator().manual_seed(0)
    mu = pkg.inputs.multinomial_lens(32, 131072, g)
    assert int(mu.sum()) == 131072 and 3500 < int(mu.min()) and int(mu.max()) < 4700


def test_quantizers(pkg, orc):
    x = torch.tensor([[0.0, 1.0], [448.0 * 3, -2.0]], dtype=torch.float32)
    q, s = pkg.inputs.quantize_tensorwise(x, "e4m3")
    assert abs(s - 3.0) < 1e-6                       # amax / 448
    assert q[1, 0].item() == 0x7E                    # the amax element maps to +448
    deq = orc.decode_e4m3(q.numpy()) * np.float32(s)
    np.testing.assert_allclose(deq, x.numpy(), rtol=2 ** -4)
    # MX: block amax 3.0 -> X = floor(log2(3/448)) = -8 -> byte 119; zero block -> 127
    xb = torch.zeros(64, 2)
    xb[:32, 0] = torch.linspace(-3.0, 3.0, 32)
    q, sc = pkg.inputs.quantize_mx(xb, "e4m3")
    assert sc.tolist() == [[119, 127], [127, 127]]
    # the recipe puts the block max in [448, 896) * 2^X, so elements beyond 448 * 2^-8 = 1.75
    # saturate (the oracle dequantizes the same bytes, so parity is unaffected)
    deq = orc.decode_e4m3(q.numpy())[:32, 0] * orc.decode_e8m0(np.array([119], np.uint8))[0]
    np.testing.assert_allclose(deq, np.clip(xb[:32, 0].numpy(), -1.75, 1.75), rtol=2 ** -3)


# ----------------------------------------------------------------------------- golden fixture

def test_golden_plumbing_fixture(pkg, orc):
    """BASELINE config 1 (G=4, M=512, groups [96,160,0,256], 64x128): the generator reproduces the
    committed bytes and the oracle reproduces the committed expected output."""
    z = np.load(os.path.join(GOLDEN, "plumbing_g4_m512.npz"))
    prob = pkg.inputs.make_problem("plumbing", seed=0, device="cpu")
    np.testing.assert_array_equal(prob.lhs.numpy(), z["lhs"])
    np.testing.assert_array_equal(prob.rhs.numpy(), z["rhs"])
    np.testing.assert_array_equal(prob.group_offs.numpy(), z["group_offs"])
    assert np.float32(prob.lhs_scale) == z["lhs_scale"] and np.float32(prob.rhs_scale) == z["rhs_scale"]
    bits = orc.vark_wgrad_tensorwise(z["lhs"], z["rhs"], z["lhs_scale"], z["rhs_scale"], z["group_offs"])
    np.testing.assert_array_equal(bits, z["expected_bf16_bits"])
    assert np.all(bits[2] == 0)
