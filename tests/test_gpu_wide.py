"""GPU parity of the wide-tile wgrad kernels (ggemm_vark_wgrad_fp8_wide: 256 x 384 and 320 x 320
tiles, one wave per SIMD, per-tile assembly from gen_vark_wide.py) against the CPU oracle, through
the C ABI.

Same bar as the other wgrad kernels: cosine >= 0.99999, max relative error <= 2e-2 over
|C| > 1e-3 * max|C|, empty groups exactly zero, no non-finite values. Cases: ragged and empty
groups (1-64-token groups, K tails of every residue class mod 64), OUT_M not a multiple of 256 (a
partial last M-tile, whose rows past OUT_M the kernel must not write), several N tiles, G up to
1100 (natural group order), offsets past M_total (clamped), a NaN-prefilled C, the full gate_up
problem compared whole, and agreement with the 192 x 384 kernel. The MXFP8 variant (320 x 320,
e8m0 block scales in the scaled MFMA) runs the MX cases: ragged groups, random fp8 codes with random
scales under the rigorous error bound, offsets past M_total, the full gate_up_mx problem against
the 192-row MX kernel.
"""
import numpy as np
import pytest
import torch

from test_gpu_parity import (_assert_parity, _assert_parity_small_k, _error_bound_ok, _oracle_whole,
                             _rand_bytes_problem)

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _run_wide(pkg, lhs, rhs, sl, sr, offs, dev, out=None, tile=True):
    return pkg.grouped_gemm_fp8_tensorwise_variable_k(
        lhs.to(dev), rhs.to(dev), torch.tensor(sl, dtype=torch.float32, device=dev),
        torch.tensor(sr, dtype=torch.float32, device=dev), offs.to(dev), out=out, wide=tile)


WIDE_CASES = [
    ([100], 256, 384, 256),
    ([1, 2, 3, 5, 8, 13, 21, 31, 63, 64, 65], 256, 384, 256),
    ([0, 0, 129, 0], 208, 384, 256),
    ([127, 128, 129, 255, 256, 257], 400, 768, 256),
    ([255, 1, 0, 256, 0, 640], 576, 1152, 256),
    ([4096 + 77], 512, 768, 256),
    ([31] * 8 + [0] * 3, 16, 384, 256),
    ([190, 191, 192, 193, 194], 2880 // 5, 1536, 256),
    ([100], 320, 320, 320),
    ([1, 2, 3, 5, 8, 13, 21, 31, 63, 64, 65], 320, 640, 320),
    ([0, 0, 129, 0], 640, 320, 320),
    ([127, 128, 129, 255, 256, 257], 960, 640, 320),
    ([255, 1, 0, 256, 0, 640], 320, 1920, 320),
    ([4096 + 77], 640, 960, 320),
    ([190, 191, 192, 193, 194], 2880 // 3, 2880 // 3, 320),
]


@pytest.mark.parametrize("lens,om,on,tile", WIDE_CASES, ids=[f"case{i}" for i in range(len(WIDE_CASES))])
def test_wide_ragged_groups_vs_oracle(pkg, orc, cuda, lens, om, on, tile):
    _say(f"wide{tile} ragged lens={lens} OUT_M={om} OUT_N={on}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=sum(lens) + om + 7)
    # NaN-prefilled C: every element must be written, rows past OUT_M of a partial tile never
    c = torch.full((len(lens), om, on), float("nan"), dtype=torch.bfloat16, device=cuda)
    out = _run_wide(pkg, lhs, rhs, sl, sr, offs, cuda, out=c, tile=tile)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
    if min(l for l in lens if l) < 40:
        _assert_parity_small_k(orc, pkg.as_bf16_bits(out), ref, lhs, rhs, offs, sl, sr, "wide/ragged")
    else:
        _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), "wide/ragged")


def test_wide_partial_tile_writes_only_its_rows(pkg, orc, cuda):
    """OUT_M = 208 inside a C whose groups are 256 rows apart (stride_cg): the 48 rows between
    groups must keep their sentinel, so the partial M-tile's rows past OUT_M are never stored."""
    lens, om, on = [64, 200, 0, 129], 208, 384
    _say(f"wide partial tile sentinel rows lens={lens}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=5)
    big = torch.full((len(lens), 256, on), 7.0, dtype=torch.bfloat16, device=cuda)
    out = _run_wide(pkg, lhs, rhs, sl, sr, offs, cuda, out=big[:, :om, :])
    torch.cuda.synchronize()
    assert bool((big[:, om:, :] == 7.0).all())
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out.contiguous()), ref, offs.numpy(), "wide/partial")


@pytest.mark.parametrize("G,tile", [(300, 256), (1100, 256), (300, 320), (1100, 320)])
def test_wide_many_groups(pkg, orc, cuda, G, tile):
    """Many small groups; G = 1100 takes the natural group order with offsets read from memory."""
    g = np.random.default_rng(G)
    lens = g.integers(0, 90, G).tolist()
    om, on = (256, 384) if tile == 256 else (320, 320)
    _say(f"wide{tile} many groups G={G} M={sum(lens)}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=G)
    out = _run_wide(pkg, lhs, rhs, sl, sr, offs, cuda, tile=tile)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
    _assert_parity_small_k(orc, pkg.as_bf16_bits(out), ref, lhs, rhs, offs, sl, sr, f"wide/G{G}")


@pytest.mark.parametrize("tile", [256, 320])
def test_wide_offsets_past_token_count_are_clamped(pkg, orc, cuda, tile):
    M = 457
    offs = torch.tensor([-64, 100, 100, 400, 600, 800], dtype=torch.int64)
    clamped = offs.clamp(min=0, max=M)
    _say(f"wide{tile} offsets past M_total: M={M} offs={offs.tolist()}")
    lens = torch.diff(clamped).tolist()
    om, on = (256, 384) if tile == 256 else (320, 640)
    lhs, rhs, _, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=43)
    pad = 512
    lhs_full = torch.cat([lhs, torch.full((pad, lhs.shape[1]), 0x38, dtype=torch.uint8)])
    rhs_full = torch.cat([rhs, torch.full((pad, rhs.shape[1]), 0x38, dtype=torch.uint8)])
    dl, dr = lhs_full.to(cuda)[:M], rhs_full.to(cuda)[:M]
    out = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, torch.tensor(sl, device=cuda), torch.tensor(sr, device=cuda),
                                                     offs.to(cuda), wide=tile)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, clamped.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, clamped.numpy(), "wide/clamp")


@pytest.mark.parametrize("om,on,tile", [(256, 352, True), (256, 320, 256), (256, 384, 320), (320, 336, 320)])
def test_wide_rejects_unsupported_shapes(pkg, cuda, om, on, tile):
    lhs = torch.zeros((64, om), dtype=torch.uint8, device=cuda)
    rhs = torch.zeros((64, on), dtype=torch.uint8, device=cuda)
    one = torch.tensor(1.0, device=cuda)
    offs = torch.tensor([0, 64], dtype=torch.int64, device=cuda)
    with pytest.raises(Exception, match="ggemm_vark_wgrad_fp8_wide"):
        pkg.grouped_gemm_fp8_tensorwise_variable_k(lhs, rhs, one, one, offs, wide=tile)


@pytest.mark.parametrize("name,tile", [("gate_up_wgrad", 256), ("gate_up_reference_lens", 256),
                                       ("gate_up_wgrad", 320), ("gate_up_reference_lens", 320), ("down_wgrad", 320)])
def test_wide_full_size(pkg, orc, cuda, name, tile):
    """Full-size problems on the wide kernels: deterministic, the whole C against the oracle, and
    within the bar of the 192-row-tile kernel's output (mfma="k32" forces that kernel)."""
    _say(f"wide{tile} full-size {name}")
    if name == "gate_up_reference_lens":
        p = pkg.inputs.make_problem("gate_up_wgrad", seed=0, device=cuda, lens=pkg.inputs.make_group_lens_reference())
    else:
        p = pkg.inputs.make_problem(name, seed=0, device=cuda)
    sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=cuda)
    sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=cuda)
    run = lambda: pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs, wide=tile)
    out = run()
    out2 = run()
    narrow = pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs, mfma="k32")
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "non-deterministic output"
    assert bool(torch.isfinite(out).all())
    m = orc.compare(pkg.as_bf16_bits(out), pkg.as_bf16_bits(narrow), p.group_offs.cpu().numpy())
    _say(f"{name}: wide{tile} vs the 192-row-tile kernel: {m}")
    assert orc.parity_ok(m)
    _oracle_whole(pkg, orc, p, out)


@pytest.mark.parametrize("lens,om,on", [([127, 128, 0, 255, 256, 257], 320, 640), ([300, 0, 645], 640, 960),
                                        ([31] * 4 + [0] * 2, 320, 320)], ids=["ragged", "two_groups", "tiny"])
def test_wide_fp32_output_and_accumulate(pkg, orc, cuda, lens, om, on):
    """The 320 x 320 kernel's fp32 epilogues: fp32 C against the float64 oracle with the bar, empty
    groups exact zeros over a NaN prefill, bf16 rounding of the fp32 result equal to the kernel's
    bf16 output bit for bit, and accumulation equal to C0 + the fp32 result exactly, twice."""
    from test_gpu_parity import _f32_parity
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=len(lens) + om + 3)
    G = len(lens)
    _say(f"wide320 fp32 out lens={lens} {om}x{on}")
    ref = orc.vark_wgrad_tensorwise_f32(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy(), acc_dtype=np.float64)
    dl, dr, do = lhs.to(cuda), rhs.to(cuda), offs.to(cuda)
    s1 = torch.tensor(sl, dtype=torch.float32, device=cuda)
    s2 = torch.tensor(sr, dtype=torch.float32, device=cuda)
    run = pkg.grouped_gemm_fp8_tensorwise_variable_k
    out = torch.full((G, om, on), float("nan"), dtype=torch.float32, device=cuda)
    run(dl, dr, s1, s2, do, out=out, out_dtype=torch.float32, wide=320)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    _f32_parity(orc, got, ref, "wide320 fp32 out")
    for g, L in enumerate(lens):
        if L == 0:
            assert np.all(got[g] == 0), g
    bf = run(dl, dr, s1, s2, do, wide=320)
    torch.cuda.synchronize()
    assert torch.equal(out.to(torch.bfloat16).view(torch.int16), bf.view(torch.int16))
    c0 = torch.randn((G, om, on), generator=torch.Generator().manual_seed(5)).float()
    acc = c0.to(cuda)
    run(dl, dr, s1, s2, do, out=acc, accumulate=True, wide=320)
    torch.cuda.synchronize()
    got1 = acc.cpu().numpy()
    np.testing.assert_array_equal(got1, (c0.numpy() + got).astype(np.float32))
    run(dl, dr, s1, s2, do, out=acc, accumulate=True, wide=320)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), (got1 + got).astype(np.float32))


@pytest.mark.parametrize("kind", ["f32", "f32_acc"])
def test_wide_fp32_offsets_clamped_and_partial_rows(pkg, orc, cuda, kind):
    """fp32 modes with offsets past M_total (clamped; extra rows hold 0x38) inside a C whose groups
    are 384 rows apart: the rows between groups keep their sentinel."""
    M = 457
    offs = torch.tensor([-64, 100, 100, 400, 600, 800], dtype=torch.int64)
    clamped = offs.clamp(min=0, max=M)
    lens = torch.diff(clamped).tolist()
    om, on = 320, 640
    _say(f"wide320 {kind} clamped offsets, strided C")
    lhs, rhs, _, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=44)
    pad = 512
    dl = torch.cat([lhs, torch.full((pad, om), 0x38, dtype=torch.uint8)]).to(cuda)[:M]
    dr = torch.cat([rhs, torch.full((pad, on), 0x38, dtype=torch.uint8)]).to(cuda)[:M]
    big = torch.full((len(lens), 384, on), 7.0, dtype=torch.float32, device=cuda)
    c0 = torch.randn((len(lens), om, on), generator=torch.Generator().manual_seed(2)).float()
    if kind == "f32_acc":
        big[:, :om, :] = c0.to(cuda)
    view = big[:, :om, :]
    pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, torch.tensor(sl, device=cuda), torch.tensor(sr, device=cuda),
                                               offs.to(cuda), out=view, out_dtype=torch.float32,
                                               accumulate=kind == "f32_acc", wide=320)
    torch.cuda.synchronize()
    assert bool((big[:, om:, :] == 7.0).all())
    from test_gpu_parity import _f32_parity
    ref = orc.vark_wgrad_tensorwise_f32(lhs.numpy(), rhs.numpy(), sl, sr, clamped.numpy(), acc_dtype=np.float64)
    got = view.cpu().numpy() - (c0.numpy() if kind == "f32_acc" else 0)
    _f32_parity(orc, got, ref, f"wide320 {kind} clamped")


# ----------------------------------------------------------------------------- MXFP8, 320 x 320

MX_WIDE_CASES = [
    ([64, 0, 96, 45], 320, 320),
    ([32] * 5 + [0, 128, 256], 640, 320),
    ([512, 0, 64, 33], 320, 960),
    ([32, 64, 96, 128, 160, 192, 224, 257], 960, 640),
    ([4096 + 64, 7], 640, 640),
]


def _run_mx(pkg, lhs, rhs, sc, offs, dev, out=None, tile_m=320):
    return pkg.grouped_gemm_mxfp8_variable_k(lhs.to(dev), rhs.to(dev), sc[0].to(dev), sc[1].to(dev), offs.to(dev),
                                             out=out, validate=True, tile_m=tile_m)


@pytest.mark.parametrize("lens,om,on", MX_WIDE_CASES, ids=[f"mx{i}" for i in range(len(MX_WIDE_CASES))])
def test_wide_mx_vs_oracle(pkg, orc, cuda, lens, om, on):
    _say(f"wide320 mx lens={lens} OUT_M={om} OUT_N={on}")
    lhs, rhs, offs, sc, _ = _rand_bytes_problem(lens, om, on, seed=sum(lens) + om + 11, mx=True)
    c = torch.full((len(lens), om, on), float("nan"), dtype=torch.bfloat16, device=cuda)
    out = _run_mx(pkg, lhs, rhs, sc, offs, cuda, out=c)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_mxfp8(lhs.numpy(), rhs.numpy(), sc[0].numpy(), sc[1].numpy(), offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), "wide/mx")


@pytest.mark.parametrize("on", [320, 1920])
def test_wide_mx_all_codes_random_scales(pkg, orc, cuda, on):
    """Uniformly random finite fp8 codes and random e8m0 scales (2^-7 .. 2^7): every element within
    the rigorous error bound of the exact block-scaled product."""
    lens = [96, 0, 64, 160, 33]
    _say(f"wide320 mx all-codes random scales OUT_N={on}")
    lhs, rhs, offs, (sl, sr), _ = _rand_bytes_problem(lens, 320, on, seed=12, mx=True, dist="codes")
    out = _run_mx(pkg, lhs, rhs, (sl, sr), offs, cuda)
    torch.cuda.synchronize()
    _error_bound_ok(orc, pkg.as_bf16_bits(out), lhs, rhs, offs, 1.0, 1.0, "wide mx codes", lsc=sl, rsc=sr)


def test_wide_mx_offsets_past_token_count_are_clamped(pkg, orc, cuda):
    """As the 192-row MX kernel's test: rows and scale rows past M_total hold 0x38 / 127, so any
    read past the token count changes the result."""
    M = 448
    offs = torch.tensor([0, 96, 96, 384, 640, 800], dtype=torch.int64)
    clamped = offs.clamp(min=0, max=M)
    _say(f"wide320 mx offsets past M_total: M={M} offs={offs.tolist()}")
    lens = torch.diff(clamped).tolist()
    lhs, rhs, _, sc, _ = _rand_bytes_problem(lens, 320, 640, seed=45, mx=True)
    pad = 512
    lhs_full = torch.cat([lhs, torch.full((pad, lhs.shape[1]), 0x38, dtype=torch.uint8)])
    rhs_full = torch.cat([rhs, torch.full((pad, rhs.shape[1]), 0x38, dtype=torch.uint8)])
    lsc = torch.cat([sc[0], torch.full((pad // 32, sc[0].shape[1]), 127, dtype=torch.uint8)])
    rsc = torch.cat([sc[1], torch.full((pad // 32, sc[1].shape[1]), 127, dtype=torch.uint8)])
    out = pkg.grouped_gemm_mxfp8_variable_k(lhs_full.to(cuda)[:M], rhs_full.to(cuda)[:M], lsc.to(cuda)[:M // 32],
                                            rsc.to(cuda)[:M // 32], offs.to(cuda), tile_m=320)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_mxfp8(lhs.numpy(), rhs.numpy(), sc[0].numpy(), sc[1].numpy(), clamped.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, clamped.numpy(), "wide/mx clamp")


def test_wide_mx_rejects_unsupported_shapes(pkg, cuda):
    lhs = torch.zeros((64, 320), dtype=torch.uint8, device=cuda)
    rhs = torch.zeros((64, 336), dtype=torch.uint8, device=cuda)
    sl = torch.full((2, 320), 127, dtype=torch.uint8, device=cuda)
    sr = torch.full((2, 336), 127, dtype=torch.uint8, device=cuda)
    offs = torch.tensor([0, 64], dtype=torch.int64, device=cuda)
    with pytest.raises(Exception, match="ggemm_vark_wgrad_mxfp8_tile"):
        pkg.grouped_gemm_mxfp8_variable_k(lhs, rhs, sl, sr, offs, tile_m=320)


def test_wide_mx_full_size(pkg, orc, cuda):
    """gate_up_mx at full size: the library picks the wide MX kernel; deterministic, the whole C
    against the oracle, and within the bar of the 192-row MX kernel (same scaled 32x32x64 MFMA
    sequence per block, so normally bit-identical)."""
    _say("wide320 mx full-size gate_up_mx")
    p = pkg.inputs.make_problem("gate_up_mx", seed=0, device=cuda)
    assert pkg.bf16_kernel(p.OUT_M, p.OUT_N) == "wide320"
    run = lambda t: pkg.grouped_gemm_mxfp8_variable_k(p.lhs, p.rhs, p.lhs_mx, p.rhs_mx, p.group_offs, tile_m=t)
    out = run(0)
    out2 = run(320)
    narrow = run(192)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "non-deterministic output"
    assert bool(torch.isfinite(out).all())
    same = float((out.view(torch.int16) == narrow.view(torch.int16)).float().mean())
    _say(f"gate_up_mx: wide vs 192-row kernel bit-identical fraction {same:.6f}")
    m = orc.compare(pkg.as_bf16_bits(out), pkg.as_bf16_bits(narrow))
    _say(f"gate_up_mx: wide vs 192-row kernel {m}")
    assert orc.parity_ok(m)
    _oracle_whole(pkg, orc, p, out)


# ----------------------------------------------------------------------------- C row strides

STRIDE_CASES = [
    # (OUT_M, OUT_N, extra columns per C row, kernel the library picks)
    (1280, 1920, 8, "wide320"), (1280, 1920, 4, "192-row"), (1024, 768, 8, "wide256"), (1024, 768, 4, "192-row"),
]


@pytest.mark.parametrize("om,on,pad,kernel", STRIDE_CASES, ids=[f"{k}_pad{p}_{m}x{n}" for m, n, p, k in STRIDE_CASES])
def test_strided_c_rows_bf16(pkg, orc, cuda, om, on, pad, kernel):
    """bf16 C rows padded by `pad` columns (stride_cm = OUT_N + pad) at shapes a wide kernel takes:
    rows on 16 bytes (pad 8) keep the wide kernel, rows on 8 bytes (pad 4) go to the 192-row kernel
    (the wide epilogue stores 16-byte row chunks). Either way the result meets the bar against the
    oracle and the padding columns keep their sentinel."""
    lens = [300, 0, 517, 64]
    _say(f"strided bf16 C {om}x{on} pad {pad}: {kernel}")
    assert pkg.bf16_kernel(om, on, on + pad) == kernel
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=om + pad)
    big = torch.full((len(lens), om, on + pad), 7.0, dtype=torch.bfloat16, device=cuda)
    out = pkg.grouped_gemm_fp8_tensorwise_variable_k(lhs.to(cuda), rhs.to(cuda), torch.tensor(sl, device=cuda),
                                                     torch.tensor(sr, device=cuda), offs.to(cuda),
                                                     out=big[:, :, :on])
    torch.cuda.synchronize()
    assert bool((big[:, :, on:] == 7.0).all())
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), f"strided bf16 pad {pad}")


@pytest.mark.parametrize("pad", [4, 8])
def test_strided_c_rows_fp32_accumulate(pkg, cuda, pad):
    """fp32 accumulate into C rows padded by `pad` floats (16-byte rows: the 320 x 320 kernel): C
    equals C0 + the contiguous fp32 result bit for bit, padding columns untouched."""
    lens, om, on = [300, 0, 517, 64], 1280, 1920
    _say(f"strided fp32-accumulate C pad {pad}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=pad + 1)
    dl, dr, do = lhs.to(cuda), rhs.to(cuda), offs.to(cuda)
    s1, s2 = torch.tensor(sl, device=cuda), torch.tensor(sr, device=cuda)
    res = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, do, out_dtype=torch.float32)
    c0 = torch.randn((len(lens), om, on), generator=torch.Generator().manual_seed(pad), dtype=torch.float32).to(cuda)
    big = torch.full((len(lens), om, on + pad), 7.0, dtype=torch.float32, device=cuda)
    big[:, :, :on] = c0
    pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, do, out=big[:, :, :on], accumulate=True)
    torch.cuda.synchronize()
    assert bool((big[:, :, on:] == 7.0).all())
    assert torch.equal(big[:, :, :on], c0 + res)


@pytest.mark.parametrize("pad,kernel", [(8, "wide320"), (4, "192-row")])
def test_strided_c_rows_mx(pkg, orc, cuda, pad, kernel):
    """The MX wgrad with bf16 C rows padded by `pad` columns: the library's choice (wide kernel for
    16-byte rows), the bar against the oracle, padding untouched."""
    lens, om, on = [64, 0, 96, 45], 1280, 1920
    _say(f"strided mx C pad {pad}: {kernel}")
    assert pkg.bf16_kernel(om, on, on + pad) == kernel
    lhs, rhs, offs, sc, _ = _rand_bytes_problem(lens, om, on, seed=pad + 17, mx=True)
    big = torch.full((len(lens), om, on + pad), 7.0, dtype=torch.bfloat16, device=cuda)
    out = _run_mx(pkg, lhs, rhs, sc, offs, cuda, out=big[:, :, :on], tile_m=0)
    torch.cuda.synchronize()
    assert bool((big[:, :, on:] == 7.0).all())
    ref = orc.vark_wgrad_mxfp8(lhs.numpy(), rhs.numpy(), sc[0].numpy(), sc[1].numpy(), offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), f"strided mx pad {pad}")


def test_forced_wide_rejects_8_byte_rows(pkg, cuda):
    lhs = torch.zeros((64, 1280), dtype=torch.uint8, device=cuda)
    rhs = torch.zeros((64, 1920), dtype=torch.uint8, device=cuda)
    one = torch.tensor(1.0, device=cuda)
    offs = torch.tensor([0, 64], dtype=torch.int64, device=cuda)
    big = torch.zeros((1, 1280, 1924), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(Exception, match="GGEMM_E_ALIGN"):
        pkg.grouped_gemm_fp8_tensorwise_variable_k(lhs, rhs, one, one, offs, out=big[:, :, :1920], wide=320)


# ----------------------------------------------------------------------------- seeded random shapes

WIDE_RANDOM_MODES = ("wide256 bf16", "wide320 bf16", "wide320 fp32", "wide320 fp32 accumulate")


@pytest.mark.parametrize("seed", range(12))
def test_wide_random_shapes_vs_oracle(pkg, orc, cuda, seed):
    """Seeded random configurations on each wide-tile kernel, forced: 256 x 384 (bf16 C) and
    320 x 320 (bf16, fp32 and fp32-accumulate C) in turn. G in 1..24 with empty, tiny (1-63 token)
    and longer groups, now and then one of 1500-3000 tokens; OUT_M and OUT_N 1-4 and 1-6 tiles of
    320, or OUT_M any multiple of 16 up to 1024 (a partial last M-tile) and 1-4 tiles of 384; LHS
    and RHS row strides padded by 0, 16 or 64 bytes; C a view into a buffer with 0 or 16 bytes of
    padding per row and 0 or 16 spare rows per group, which keep their sentinel. bf16 C: the bar
    against the oracle, or, when a group is shorter than 40 tokens, the bar's cosine, finiteness
    and exact-zero empty groups plus every element within the rigorous fp8-MFMA error bound. fp32
    C: the bar on fp32 values, or the cosine plus the bound without output rounding.
    Accumulation: C0 + the fp32 result, bit for bit."""
    rng = np.random.default_rng(7000 + seed)
    mode = WIDE_RANDOM_MODES[seed % 4]
    tile = 256 if mode.startswith("wide256") else 320
    fp32 = "fp32" in mode
    G = int(rng.integers(1, 25))
    kind = rng.integers(0, 4, G)
    lens = np.where(kind == 0, 0, np.where(kind == 1, rng.integers(1, 64, G), rng.integers(64, 700, G)))
    if seed % 3 == 0:
        lens[rng.integers(0, G)] = int(rng.integers(1500, 3001))
    lens = [int(v) for v in lens]
    if tile == 320:
        om, on = 320 * int(rng.integers(1, 5)), 320 * int(rng.integers(1, 7))
    else:
        om, on = 16 * int(rng.integers(1, 65)), 384 * int(rng.integers(1, 5))
    lpad, rpad = int(rng.choice([0, 16, 64])), int(rng.choice([0, 16, 64]))
    esize = 4 if fp32 else 2
    cpad = int(rng.choice([0, 16])) // esize
    rows_extra = int(rng.choice([0, 16]))
    M = sum(lens)
    _say(f"wide random seed={seed} {mode} G={G} M={M} OUT={om}x{on} lhs/rhs pad {lpad}/{rpad} B, "
         f"C pad {cpad} cols {rows_extra} rows")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=seed + 91)
    dl = torch.zeros((max(M, 1), om + lpad), dtype=torch.uint8, device=cuda)[:M, :om]
    dl.copy_(lhs)
    dr = torch.zeros((max(M, 1), on + rpad), dtype=torch.uint8, device=cuda)[:M, :on]
    dr.copy_(rhs)
    do = offs.to(cuda)
    s1 = torch.tensor(sl, dtype=torch.float32, device=cuda)
    s2 = torch.tensor(sr, dtype=torch.float32, device=cuda)
    dt = torch.float32 if fp32 else torch.bfloat16
    big = torch.full((G, om + rows_extra, on + cpad), 7.0, dtype=dt, device=cuda)
    view = big[:, :om, :on]
    view.fill_(float("nan"))
    run = pkg.grouped_gemm_fp8_tensorwise_variable_k
    run(dl, dr, s1, s2, do, out=view, out_dtype=dt, wide=tile)
    torch.cuda.synchronize()
    assert bool((big[:, om:, :] == 7.0).all()) and bool((big[:, :, on:] == 7.0).all())
    tiny = any(0 < v < 40 for v in lens)
    if not fp32:
        ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
        bits = pkg.as_bf16_bits(view)
        if tiny:
            _assert_parity_small_k(orc, bits, ref, lhs, rhs, offs, sl, sr, f"wide random {seed}")
        else:
            _assert_parity(orc, bits, ref, offs.numpy(), f"wide random {seed}")
        return
    got = view.cpu().numpy()
    for g, v in enumerate(lens):
        if v == 0:
            assert np.all(got[g] == 0), g
    ref = orc.vark_wgrad_tensorwise_f32(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy(), acc_dtype=np.float64)
    a, b = got.astype(np.float64).ravel(), ref.astype(np.float64).ravel()
    assert np.isfinite(a).all()
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300)) if M else 1.0
    mask = np.abs(b) > 1e-3 * np.abs(b).max() if M else np.zeros(b.shape, bool)
    rel = float(np.max(np.abs(a[mask] - b[mask]) / np.abs(b[mask]))) if mask.any() else 0.0
    _say(f"wide random {seed} fp32: cos {cos:.9f} max_rel {rel:.3e}")
    assert cos >= 0.99999, (seed, cos)
    if rel > 2e-2:
        viol, worst = orc.mfma_bound_violations(got, lhs.numpy(), rhs.numpy(), offs.numpy(), sl, sr,
                                                out_rounding=0.0)
        _say(f"wide random {seed} fp32: error-bound violations {int(viol.sum())}, worst ratio {worst:.3f}")
        assert not viol.any()
    if mode.endswith("accumulate"):
        c0 = torch.randn((G, om, on), generator=torch.Generator().manual_seed(seed), dtype=torch.float32)
        view.copy_(c0.to(cuda))
        run(dl, dr, s1, s2, do, out=view, accumulate=True, wide=tile)
        torch.cuda.synchronize()
        assert bool((big[:, om:, :] == 7.0).all()) and bool((big[:, :, on:] == 7.0).all())
        np.testing.assert_array_equal(view.cpu().numpy(), (c0.numpy() + got).astype(np.float32))


@pytest.mark.parametrize("seed", range(6))
def test_wide_mx_random_shapes_vs_oracle(pkg, orc, cuda, seed):
    """Seeded random configurations on the wide MX kernel (forced, tile_m=320): G in 1..16 with
    empty groups and groups of 32-640 tokens in whole 32-token blocks, the last group of any
    length; OUT_M and OUT_N 1-4 and 1-6 tiles of 320; LHS / RHS row strides padded by 0, 16 or 64
    bytes and the e8m0 scale rows by 16 on odd seeds; C a view with 8 columns of padding per row,
    which keep their sentinel. The bar against the oracle, or its cosine, finiteness and
    exact-zero empty groups plus every element within the rigorous error bound of the
    block-scaled product."""
    rng = np.random.default_rng(8000 + seed)
    G = int(rng.integers(1, 17))
    blocks = np.where(rng.integers(0, 4, G) == 0, 0, rng.integers(1, 21, G))
    lens = [32 * int(v) for v in blocks]
    lens[-1] = int(rng.integers(1, 700))
    om, on = 320 * int(rng.integers(1, 5)), 320 * int(rng.integers(1, 7))
    lpad, rpad = int(rng.choice([0, 16, 64])), int(rng.choice([0, 16, 64]))
    spad = 16 * (seed % 2)
    _say(f"wide mx random seed={seed} G={G} M={sum(lens)} OUT={om}x{on} lhs/rhs pad {lpad}/{rpad} B, "
         f"scale pad {spad} B")
    lhs, rhs, offs, (sl, sr), _ = _rand_bytes_problem(lens, om, on, seed=seed + 37, mx=True)

    def padded(t, pad):
        v = torch.zeros((max(t.shape[0], 1), t.shape[1] + pad), dtype=torch.uint8, device=cuda)
        v = v[:t.shape[0], :t.shape[1]]
        v.copy_(t)
        return v

    big = torch.full((G, om, on + 8), 7.0, dtype=torch.bfloat16, device=cuda)
    view = big[:, :, :on]
    view.fill_(float("nan"))
    pkg.grouped_gemm_mxfp8_variable_k(padded(lhs, lpad), padded(rhs, rpad), padded(sl, spad), padded(sr, spad),
                                      offs.to(cuda), out=view, validate=True, tile_m=320)
    torch.cuda.synchronize()
    assert bool((big[:, :, on:] == 7.0).all())
    ref = orc.vark_wgrad_mxfp8(lhs.numpy(), rhs.numpy(), sl.numpy(), sr.numpy(), offs.numpy())
    bits = pkg.as_bf16_bits(view)
    m = orc.compare(bits, ref, offs.numpy())
    _say(f"wide mx random {seed}: {m}")
    if not orc.parity_ok(m):
        assert m["cos"] >= 0.99999 and m["nonfinite"] == 0 and m["empty_zero"], (seed, m)
        _error_bound_ok(orc, bits, lhs, rhs, offs, 1.0, 1.0, f"wide mx random {seed}", lsc=sl, rsc=sr)
