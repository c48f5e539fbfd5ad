"""GPU parity of the wide-tile wgrad kernel (ggemm_vark_wgrad_fp8_wide: 256 x 384 tiles, one wave
per SIMD, per-tile assembly from gen_vark_wide.py) against the CPU oracle, through the C ABI.

Same bar as the other wgrad kernels: cosine >= 0.99999, max relative error <= 2e-2 over
|C| > 1e-3 * max|C|, empty groups exactly zero, no non-finite values. Cases: ragged and empty
groups (1-64-token groups, K tails of every residue class mod 64), OUT_M not a multiple of 256 (a
partial last M-tile, whose rows past OUT_M the kernel must not write), several N tiles, G up to
1100 (natural group order), offsets past M_total (clamped), a NaN-prefilled C, the full gate_up
problem compared whole, and agreement with the 192 x 384 kernel.
"""
import numpy as np
import pytest
import torch

from test_gpu_parity import _assert_parity, _assert_parity_small_k, _oracle_whole, _rand_bytes_problem

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _run_wide(pkg, lhs, rhs, sl, sr, offs, dev, out=None):
    return pkg.grouped_gemm_fp8_tensorwise_variable_k(
        lhs.to(dev), rhs.to(dev), torch.tensor(sl, dtype=torch.float32, device=dev),
        torch.tensor(sr, dtype=torch.float32, device=dev), offs.to(dev), out=out, wide=True)


WIDE_CASES = [
    ([100], 256, 384),
    ([1, 2, 3, 5, 8, 13, 21, 31, 63, 64, 65], 256, 384),
    ([0, 0, 129, 0], 208, 384),
    ([127, 128, 129, 255, 256, 257], 400, 768),
    ([255, 1, 0, 256, 0, 640], 576, 1152),
    ([4096 + 77], 512, 768),
    ([31] * 8 + [0] * 3, 16, 384),
    ([190, 191, 192, 193, 194], 2880 // 5, 1536),
]


@pytest.mark.parametrize("lens,om,on", WIDE_CASES, ids=[f"case{i}" for i in range(len(WIDE_CASES))])
def test_wide_ragged_groups_vs_oracle(pkg, orc, cuda, lens, om, on):
    _say(f"wide ragged lens={lens} OUT_M={om} OUT_N={on}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=sum(lens) + om + 7)
    # NaN-prefilled C: every element must be written, rows past OUT_M of a partial tile never
    c = torch.full((len(lens), om, on), float("nan"), dtype=torch.bfloat16, device=cuda)
    out = _run_wide(pkg, lhs, rhs, sl, sr, offs, cuda, out=c)
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


@pytest.mark.parametrize("G", [300, 1100])
def test_wide_many_groups(pkg, orc, cuda, G):
    """Many small groups; G = 1100 takes the natural group order with offsets read from memory."""
    g = np.random.default_rng(G)
    lens = g.integers(0, 90, G).tolist()
    _say(f"wide many groups G={G} M={sum(lens)}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, 256, 384, seed=G)
    out = _run_wide(pkg, lhs, rhs, sl, sr, offs, cuda)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
    _assert_parity_small_k(orc, pkg.as_bf16_bits(out), ref, lhs, rhs, offs, sl, sr, f"wide/G{G}")


def test_wide_offsets_past_token_count_are_clamped(pkg, orc, cuda):
    M = 457
    offs = torch.tensor([-64, 100, 100, 400, 600, 800], dtype=torch.int64)
    clamped = offs.clamp(min=0, max=M)
    _say(f"wide offsets past M_total: M={M} offs={offs.tolist()}")
    lens = torch.diff(clamped).tolist()
    lhs, rhs, _, _, (sl, sr) = _rand_bytes_problem(lens, 256, 384, seed=43)
    pad = 512
    lhs_full = torch.cat([lhs, torch.full((pad, lhs.shape[1]), 0x38, dtype=torch.uint8)])
    rhs_full = torch.cat([rhs, torch.full((pad, rhs.shape[1]), 0x38, dtype=torch.uint8)])
    dl, dr = lhs_full.to(cuda)[:M], rhs_full.to(cuda)[:M]
    out = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, torch.tensor(sl, device=cuda), torch.tensor(sr, device=cuda),
                                                     offs.to(cuda), wide=True)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, clamped.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, clamped.numpy(), "wide/clamp")


def test_wide_rejects_unsupported_shapes(pkg, cuda):
    lhs = torch.zeros((64, 256), dtype=torch.uint8, device=cuda)
    rhs = torch.zeros((64, 320), dtype=torch.uint8, device=cuda)
    one = torch.tensor(1.0, device=cuda)
    offs = torch.tensor([0, 64], dtype=torch.int64, device=cuda)
    with pytest.raises(Exception, match="ggemm_vark_wgrad_fp8_wide"):
        pkg.grouped_gemm_fp8_tensorwise_variable_k(lhs, rhs, one, one, offs, wide=True)


@pytest.mark.parametrize("name", ["gate_up_wgrad", "gate_up_reference_lens"])
def test_wide_full_size(pkg, orc, cuda, name):
    """The full gate_up problem on the wide kernel: deterministic, the whole C against the oracle,
    and within the bar of the 192 x 384 kernel's output."""
    _say(f"wide full-size {name}")
    if name == "gate_up_reference_lens":
        p = pkg.inputs.make_problem("gate_up_wgrad", seed=0, device=cuda, lens=pkg.inputs.make_group_lens_reference())
    else:
        p = pkg.inputs.make_problem(name, seed=0, device=cuda)
    sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=cuda)
    sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=cuda)
    run = lambda: pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs, wide=True)
    out = run()
    out2 = run()
    narrow = pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "non-deterministic output"
    assert bool(torch.isfinite(out).all())
    m = orc.compare(pkg.as_bf16_bits(out), pkg.as_bf16_bits(narrow), p.group_offs.cpu().numpy())
    _say(f"{name}: wide vs 192x384 kernel: {m}")
    assert orc.parity_ok(m)
    _oracle_whole(pkg, orc, p, out)
