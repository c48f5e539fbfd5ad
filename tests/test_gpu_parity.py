"""GPU parity of the HIP kernels against the CPU oracle (all launches through the C ABI or the
drop-in code object).

Bar (from the north-star statement): cosine >= 0.99999, max relative error <= 2e-2 over
|C| > 1e-3 * max|C|, empty groups exactly zero, no non-finite values. Every case, the full-size
configurations included, compares its whole output with the oracle; the full-size ones also check
the size-independent row-sum and column-sum identities
``C[g] @ 1 = sL*sR * LHS_g^T (RHS_g @ 1)`` and ``1^T C[g] = sL*sR * (1^T LHS_g^T) RHS_g`` on every
row and column of every group.
"""
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from conftest import GOLDEN, ROOT

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _rand_bytes_problem(lens, om, on, seed, mx=False, dist="normal"):
    """CPU-generated problem. dist="normal": the measured configurations' value distributions
    (LHS N(0,1) -> e4m3 with amax/448, RHS N(0,1e-3) -> e5m2 with amax/57344; MX: e8m0 block scales
    by the same recipe, token count padded to a multiple of 32 with zero rows). dist="codes":
    uniformly random finite fp8 codes (full exponent range) and random e8m0 scales."""
    g = torch.Generator().manual_seed(seed)
    M = int(sum(lens))
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    if dist == "codes":
        lhs = torch.randint(0, 256, (M, om), generator=g, dtype=torch.int32).to(torch.uint8)
        rhs = torch.randint(0, 256, (M, on), generator=g, dtype=torch.int32).to(torch.uint8)
        lhs[(lhs & 0x7F) == 0x7F] = 0x3A       # e4m3fn NaN codes -> 1.25
        rhs[(rhs & 0x7C) == 0x7C] = 0x3B       # e5m2 inf/NaN codes -> 0.875
        sc = None
        if mx:
            nb = (M + 31) // 32
            sc = (torch.randint(120, 135, (nb, om), generator=g, dtype=torch.int32).to(torch.uint8),
                  torch.randint(120, 135, (nb, on), generator=g, dtype=torch.int32).to(torch.uint8))
        return lhs, rhs, offs, sc, (0.0173, 2.9e-4)
    from ggemm_asm_amd import inputs
    if M == 0:
        return (torch.zeros((0, om), dtype=torch.uint8), torch.zeros((0, on), dtype=torch.uint8), offs, None,
                (1.0, 1.0))
    Mp = (M + 31) // 32 * 32 if mx else M
    x = torch.randn((Mp, om), generator=g)
    dy = torch.randn((Mp, on), generator=g) * 1e-3
    x[M:] = 0
    dy[M:] = 0
    if mx:
        lhs, sl = inputs.quantize_mx(x, "e4m3")
        rhs, sr = inputs.quantize_mx(dy, "e5m2")
        return lhs, rhs, offs, (sl, sr), (1.0, 1.0)
    lhs, sl = inputs.quantize_tensorwise(x[:M], "e4m3")
    rhs, sr = inputs.quantize_tensorwise(dy[:M], "e5m2")
    return lhs, rhs, offs, None, (sl, sr)


def _error_bound_ok(orc, got_bits, lhs, rhs, offs, sl, sr, label, lsc=None, rsc=None):
    """Rigorous check for adversarial inputs (oracle.mfma_bound_violations, pinned on the CPU by
    tests/test_oracle_mfma.py): |got - exact| <= 2^-8 |exact| (bf16 output rounding) + the fp8-MFMA
    accumulation bound + fp32 scale rounding, on every element."""
    viol, worst = orc.mfma_bound_violations(
        orc.bf16_bits_to_f32(got_bits), lhs.numpy(), rhs.numpy(), offs.numpy(), sl, sr,
        None if lsc is None else lsc.numpy(), None if rsc is None else rsc.numpy())
    _say(f"{label}: error-bound violations {int(viol.sum())} of {viol.size}, worst ratio {worst:.3f}")
    assert not viol.any()


def _run_tw(pkg, lhs, rhs, sl, sr, offs, dev, mfma="k128"):
    return pkg.grouped_gemm_fp8_tensorwise_variable_k(
        lhs.to(dev), rhs.to(dev), torch.tensor(sl, dtype=torch.float32, device=dev),
        torch.tensor(sr, dtype=torch.float32, device=dev), offs.to(dev), mfma=mfma)


def _assert_parity(orc, got_bits, ref_bits, offs, label):
    m = orc.compare(got_bits, ref_bits, offs)
    _say(f"{label}: {m}")
    assert orc.parity_ok(m), (label, m)
    return m


def _assert_parity_small_k(orc, got_bits, ref_bits, lhs, rhs, offs, sl, sr, label):
    """The bar's cosine, finiteness and exact-zero empty groups on every element; its 2e-2 relative
    bound may be exceeded only by elements whose exact value is a heavy cancellation of much larger
    products, and every element must lie within the rigorous fp8-MFMA error bound (at K < 40 a
    block-truncated sum can be a few percent of such a result)."""
    m = orc.compare(got_bits, ref_bits, offs.numpy())
    _say(f"{label}: {m}")
    assert m["cos"] >= 0.99999 and m["nonfinite"] == 0 and m["empty_zero"], (label, m)
    _error_bound_ok(orc, got_bits, lhs, rhs, offs, sl, sr, label)


# ----------------------------------------------------------------------------- small, full compare

def test_plumbing_golden_fixture(pkg, orc, cuda):
    _say("plumbing golden G=4 M=512 64x128")
    z = np.load(os.path.join(GOLDEN, "plumbing_g4_m512.npz"))
    out = _run_tw(pkg, torch.from_numpy(z["lhs"]), torch.from_numpy(z["rhs"]), float(z["lhs_scale"]),
                  float(z["rhs_scale"]), torch.from_numpy(z["group_offs"]), cuda)
    torch.cuda.synchronize()
    m = _assert_parity(orc, pkg.as_bf16_bits(out), z["expected_bf16_bits"], z["group_offs"], "plumbing")
    assert np.all(pkg.as_bf16_bits(out)[2] == 0)
    assert m["exact_frac"] > 0.9


RAGGED = [
    ([1, 2, 3, 5, 8, 13, 21, 31], 64, 128),
    ([0, 0, 129, 0], 192, 320),
    ([127, 128, 129, 255, 256, 257], 208, 336),
    ([255, 1, 0, 256, 0, 640], 400, 656),
    ([31] * 8 + [0] * 3, 16, 16),
    ([1000, 24], 2880 // 5, 5760 // 9),
    ([0], 64, 64),
    ([4096 + 77], 384, 640),
    # OUT_N multiples of 384 take the 192 x 384 tile configuration
    ([1, 2, 3, 5, 8, 13, 21, 31], 64, 384),
    ([127, 128, 129, 0, 256, 257], 208, 768),
    ([300, 0, 645], 400, 1152),
    ([31] * 4 + [0] * 2, 16, 384),
    ([2000, 96], 576, 768),
    # OUT_N = 4.5 x 384: 384-wide tiles with a half-full last one (as at OUT_N = 2880)
    ([255, 0, 129, 640], 208, 1728),
]


@pytest.mark.parametrize("lens,om,on", RAGGED, ids=[f"case{i}" for i in range(len(RAGGED))])
@pytest.mark.parametrize("mfma", ["k128", "k32"])
def test_ragged_groups_vs_oracle(pkg, orc, cuda, lens, om, on, mfma):
    _say(f"ragged lens={lens} OUT_M={om} OUT_N={on} mfma={mfma}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=sum(lens) + om)
    out = _run_tw(pkg, lhs, rhs, sl, sr, offs, cuda, mfma)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), f"ragged/{mfma}")


@pytest.mark.parametrize("mfma", ["k128", "k32"])
def test_all_fp8_codes_error_bound(pkg, orc, cuda, mfma):
    """Uniformly random finite fp8 codes (every exponent) against the rigorous error bound."""
    _say(f"all-codes adversarial mfma={mfma}")
    lens = [1, 31, 0, 129, 300]
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, 208, 336, seed=3, dist="codes")
    out = _run_tw(pkg, lhs, rhs, sl, sr, offs, cuda, mfma)
    torch.cuda.synchronize()
    _error_bound_ok(orc, pkg.as_bf16_bits(out), lhs, rhs, offs, sl, sr, f"codes/{mfma}")


@pytest.mark.parametrize("on", [128, 384, 768])
def test_mxfp8_all_codes_random_scales(pkg, orc, cuda, on):
    """MX path with random codes and random e8m0 scales (every scale byte position of both tile
    widths), against the same rigorous bound."""
    _say(f"mxfp8 all-codes random scales OUT_N={on}")
    lens = [64, 0, 96, 32, 213]
    lhs, rhs, offs, (sl, sr), _ = _rand_bytes_problem(lens, 208, on, seed=8, mx=True, dist="codes")
    out = pkg.grouped_gemm_mxfp8_variable_k(lhs.to(cuda), rhs.to(cuda), sl.to(cuda), sr.to(cuda), offs.to(cuda))
    torch.cuda.synchronize()
    _error_bound_ok(orc, pkg.as_bf16_bits(out), lhs, rhs, offs, 1.0, 1.0, "mx codes", lsc=sl, rsc=sr)


def test_output_fully_overwritten(pkg, orc, cuda):
    """The kernel owns every element of C (launcher.cpp never re-zeroes C between launches)."""
    _say("overwrite: C pre-filled with NaN")
    lhs, rhs, offs, _, _ = _rand_bytes_problem([50, 0, 300, 7], 208, 336, seed=9)
    out = torch.full((4, 208, 336), float("nan"), dtype=torch.bfloat16, device=cuda)
    pkg.grouped_gemm_fp8_tensorwise_variable_k(
        lhs.to(cuda), rhs.to(cuda), torch.tensor(0.5, device=cuda), torch.tensor(0.25, device=cuda),
        offs.to(cuda), out=out)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), 0.5, 0.25, offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), "overwrite")


def test_strided_views(pkg, orc, cuda):
    """Row strides larger than the width and a C with padded rows/groups."""
    _say("strided views")
    lens = [100, 0, 157]
    lhs_full, rhs_full, offs, _, _ = _rand_bytes_problem(lens, 96, 160, seed=11)
    lhs = lhs_full[:, :64]
    rhs = rhs_full[:, :128]
    dl, dr = lhs_full.to(cuda)[:, :64], rhs_full.to(cuda)[:, :128]
    big = torch.zeros((3, 80, 144), dtype=torch.bfloat16, device=cuda)
    out = big[:, :64, :128]
    pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, torch.tensor(0.3, device=cuda), torch.tensor(0.7, device=cuda),
                                              offs.to(cuda), out=out)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.contiguous().numpy(), rhs.contiguous().numpy(), 0.3, 0.7, offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), "strided")
    assert torch.count_nonzero(big[:, 64:, :]) == 0 and torch.count_nonzero(big[:, :, 128:]) == 0


@pytest.mark.parametrize("seed", range(12))
def test_random_shapes_vs_oracle(pkg, orc, cuda, seed):
    """Seeded random configurations: G in 1..40 with empty, tiny and long groups; OUT_M, OUT_N any
    multiples of 16 up to 800 (partial tiles in both dimensions, both tile widths and the wide-tile
    rule's boundary), realistic values: the bar on cosine, finiteness and exact-zero empty groups,
    and its 2e-2 relative threshold, or, where a tiny group's heavy cancellation exceeds that, every
    element within the rigorous MFMA error bound."""
    rng = np.random.default_rng(1000 + seed)
    G = int(rng.integers(1, 41))
    kind = rng.integers(0, 4, G)
    lens = np.where(kind == 0, 0, np.where(kind == 1, rng.integers(1, 32, G), rng.integers(32, 400, G)))
    if seed % 3 == 0:
        lens[rng.integers(0, G)] = int(rng.integers(1000, 2500))       # one long group (skew)
    om = 16 * int(rng.integers(1, 26))
    on = 16 * int(rng.choice([int(rng.integers(1, 51)), 96, 108, 120]))  # 1536, 1728, 1920 included
    _say(f"random seed={seed} G={G} M={int(lens.sum())} OUT={om}x{on}")
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens.tolist(), om, on, seed=seed)
    out = _run_tw(pkg, lhs, rhs, sl, sr, offs, cuda)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy())
    bits = pkg.as_bf16_bits(out)
    m = orc.compare(bits, ref, offs.numpy())
    _say(f"random {seed}: {m}")
    if not orc.parity_ok(m):
        _assert_parity_small_k(orc, bits, ref, lhs, rhs, offs, sl, sr, f"random {seed}")


@pytest.mark.parametrize("G,skew", [(1100, False), (1024, False), (1024, True)])
def test_many_groups_natural_order(pkg, orc, cuda, G, skew):
    """G above the in-kernel sort limit (1024) uses natural group order; G = 1024 is the largest
    sorted case, its tile weights filling the schedule's weight table (a few long groups among
    short ones make the deals differ)."""
    _say(f"G={G} skew={skew}")
    rng = np.random.default_rng(G + skew)
    lens = rng.integers(0, 40, G)
    if skew:
        lens[rng.choice(G, 6, replace=False)] = rng.integers(600, 1500, 6)
    lens = lens.tolist()
    lhs, rhs, offs, _, _ = _rand_bytes_problem(lens, 32, 48, seed=12)
    out = _run_tw(pkg, lhs, rhs, 0.01, 0.02, offs, cuda)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), 0.01, 0.02, offs.numpy())
    _assert_parity_small_k(orc, pkg.as_bf16_bits(out), ref, lhs, rhs, offs, 0.01, 0.02, f"G={G}")


MX_CASES = [([64, 0, 96, 45], 64, 128), ([32] * 5 + [0, 128, 256], 192, 320), ([512, 0, 64], 208, 336),
            # OUT_N multiples of 384 take the 192 x 384 tile configuration
            ([64, 0, 96, 45], 64, 384), ([32] * 5 + [0, 128, 256], 400, 768), ([1024, 32], 192, 1152)]


@pytest.mark.parametrize("lens,om,on", MX_CASES, ids=[f"mx{i}" for i in range(len(MX_CASES))])
def test_mxfp8_vs_oracle(pkg, orc, cuda, lens, om, on):
    _say(f"mxfp8 lens={lens} OUT_M={om} OUT_N={on}")
    lhs, rhs, offs, (sl, sr), _ = _rand_bytes_problem(lens, om, on, seed=sum(lens) + 5, mx=True)
    out = pkg.grouped_gemm_mxfp8_variable_k(lhs.to(cuda), rhs.to(cuda), sl.to(cuda), sr.to(cuda), offs.to(cuda),
                                            validate=True)
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_mxfp8(lhs.numpy(), rhs.numpy(), sl.numpy(), sr.numpy(), offs.numpy())
    _assert_parity(orc, pkg.as_bf16_bits(out), ref, offs.numpy(), "mxfp8")


# ----------------------------------------------------------------------------- drop-in code object

@pytest.mark.parametrize("out_n", [640, 768])
def test_code_object_kernelparams_and_kernarg_buffer(pkg, cuda, out_n):
    """Our .co launched like reference bench.py (16-entry kernelParams) and like launcher.cpp
    (96-byte buffer) gives the library's result bit for bit (both N-tile configurations)."""
    from ggemm_asm_amd import harness
    _say(f"code object via hipModuleLaunchKernel OUT_N={out_n}")
    lens = [96, 160, 0, 256, 33]
    lhs, rhs, offs, _, _ = _rand_bytes_problem(lens, 384, out_n, seed=21)
    dl, dr, do = lhs.to(cuda), rhs.to(cuda), offs.to(cuda)
    s1, s2 = torch.tensor(0.1, device=cuda), torch.tensor(0.1, device=cuda)
    ref = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, do)
    module, func, name = harness.load_kernel(pkg.CODE_OBJECT_PATH)
    assert name == "_grouped_variable_k_gemm_kernel"
    try:
        n_cus = harness.get_num_cus(0)
        out1 = torch.zeros_like(ref)
        torch.cuda.synchronize()
        harness.launch_variable_k_kernel(func, dl, dr, out1, s1, s2, do, len(lens), 384, out_n, n_cus)
        out2 = torch.full_like(ref, 7.0)
        harness.launch_with_kernarg_buffer(func, harness.kernarg_buffer(dl, dr, out2, s1, s2, do, len(lens), 384, out_n),
                                           n_cus)
        torch.cuda.synchronize()
        assert torch.equal(out1.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(out2.view(torch.int16), ref.view(torch.int16))
        # any grid size must be correct: 24 spreads over the 8 XCDs (two deals to choose from), 20
        # and 1 do not (one slice); 1032 and 600 exceed the 512 threads that weigh the deals (each
        # thread weighs several workgroups), 1032 spreading over the XCDs, 600 not
        for grid in (24, 20, 1, 1032, 600):
            out3 = torch.zeros_like(ref)
            harness.launch_variable_k_kernel(func, dl, dr, out3, s1, s2, do, len(lens), 384, out_n, grid)
            torch.cuda.synchronize()
            assert torch.equal(out3.view(torch.int16), ref.view(torch.int16)), grid
    finally:
        harness.unload_kernel(module)


def test_reference_launcher_runs_code_object(pkg):
    """The reference's own launcher.cpp (compiled unmodified into oracle/_ref/) loads and times our
    code object on its constant-fill gate_up_wgrad inputs."""
    exe = os.path.join(ROOT, "oracle", "_ref", "launcher")
    if not os.path.exists(exe):
        pytest.skip("reference launcher not built (reference tree was not mounted at build time)")
    _say("reference launcher.cpp with our .co")
    r = subprocess.run([exe, pkg.CODE_OBJECT_PATH, "--site", "gate_up_wgrad", "--warmup", "20", "--iters", "50"],
                       capture_output=True, text=True, timeout=120)
    _say(r.stdout.strip().replace("\n", " | "))
    assert r.returncode == 0, r.stderr
    assert re.search(r"Site: gate_up_wgrad\s+E=32 M=131072 OUT_M=2880 OUT_N=5760", r.stdout)
    m = re.search(r"Kernel:\s+([\d.]+) ms\s+([\d.]+) TFLOPS", r.stdout)
    assert m and float(m.group(1)) > 0
    # the same code object on the same inputs, launched through the reference's hipModule path
    # (harness: kernelParams array, null stream) and timed the same way (events around 50 launches
    # after 20): the launcher must run it at the same speed, and the C it writes is the closed form
    from ggemm_asm_amd import harness
    dev = torch.device("cuda:0")
    p = pkg.inputs.constant_problem(device=dev)
    s = torch.tensor(0.1, device=dev)
    out = torch.empty((p.G, p.OUT_M, p.OUT_N), dtype=torch.bfloat16, device=dev)
    module, func, _ = harness.load_kernel(pkg.CODE_OBJECT_PATH)
    try:
        launch, _keep = harness.prepare_variable_k_args(func, p.lhs, p.rhs, out, s, s, p.group_offs, p.G, p.OUT_M,
                                                        p.OUT_N, harness.get_num_cus())
        torch.cuda.synchronize()
        co_ms = harness.time_null_stream(launch, 50, 20)
    finally:
        harness.unload_kernel(module)
    ratio = float(m.group(1)) / co_ms
    _say(f"launcher {float(m.group(1)):.3f} ms, same .co through the hipModule harness {co_ms:.3f} ms, "
         f"ratio {ratio:.3f}")
    assert bool((out.view(torch.int16) == 0x41A4).all())
    assert 0.85 < ratio < 1.15


# ----------------------------------------------------------------------------- full-size configs

def test_constant_fill_known_answer_full_size(pkg, cuda):
    """launcher.cpp:97-112 inputs at gate_up_wgrad size: every element must be 20.5 (0x41A4)."""
    _say("constant fill gate_up 32x2880x5760")
    p = pkg.inputs.constant_problem(device=cuda)
    out = pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, torch.tensor(0.1, device=cuda),
                                                     torch.tensor(0.1, device=cuda), p.group_offs)
    torch.cuda.synchronize()
    assert bool((out.view(torch.int16) == 0x41A4).all())


def _rowsum_identity(pkg, p, out, dev):
    """max over (g, m) of |sum_n C - sL sR sum_k L[k,m] (sum_n R[k,n])| / (sum_n |C| + eps)."""
    worst = 0.0
    offs = p.group_offs.cpu().tolist()
    for g in range(p.G):
        lo, hi = offs[g], offs[g + 1]
        c = out[g].float()
        lhs_rows = c.sum(dim=1).double()
        if hi == lo:
            assert bool((out[g].view(torch.int16) & 0x7FFF == 0).all())
            continue
        if p.is_mx:
            blk = torch.arange(lo, hi, device=dev) // 32
            L = p.lhs[lo:hi].view(torch.float8_e4m3fn).float() * torch.exp2(p.lhs_mx[blk].float() - 127)
            R = p.rhs[lo:hi].view(torch.float8_e5m2).float() * torch.exp2(p.rhs_mx[blk].float() - 127)
            rhs_rows = (L.double().T @ R.double().sum(dim=1))
        else:
            L = p.lhs[lo:hi].view(torch.float8_e4m3fn).double()
            R = p.rhs[lo:hi].view(torch.float8_e5m2).double()
            rhs_rows = (L.T @ R.sum(dim=1)) * p.lhs_scale * p.rhs_scale
        denom = c.abs().sum(dim=1).double() + 1e-30
        worst = max(worst, float(((lhs_rows - rhs_rows).abs() / denom).max()))
    return worst


def _colsum_identity(pkg, p, out, dev):
    """max over (g, n) of |sum_m C[m,n] - sL sR (sum_m L[k,m]) . R[k,n]| / (sum_m |C| + eps): the
    column sums pin where each OUT_N column landed (the row sums pin the OUT_M rows)."""
    worst = 0.0
    offs = p.group_offs.cpu().tolist()
    for g in range(p.G):
        lo, hi = offs[g], offs[g + 1]
        if hi == lo:
            continue
        c = out[g].float()
        lhs_cols = c.sum(dim=0).double()
        if p.is_mx:
            blk = torch.arange(lo, hi, device=dev) // 32
            L = p.lhs[lo:hi].view(torch.float8_e4m3fn).float() * torch.exp2(p.lhs_mx[blk].float() - 127)
            R = p.rhs[lo:hi].view(torch.float8_e5m2).float() * torch.exp2(p.rhs_mx[blk].float() - 127)
            rhs_cols = L.double().sum(dim=1) @ R.double()
        else:
            L = p.lhs[lo:hi].view(torch.float8_e4m3fn).double()
            R = p.rhs[lo:hi].view(torch.float8_e5m2).double()
            rhs_cols = (L.sum(dim=1) @ R) * p.lhs_scale * p.rhs_scale
        denom = c.abs().sum(dim=0).double() + 1e-30
        worst = max(worst, float(((lhs_cols - rhs_cols).abs() / denom).max()))
    return worst


def _oracle_whole(pkg, orc, p, out):
    """Every group of the full-size output against the oracle, with the bar over the whole tensor
    (cosine over all of C, the 1e-3 * max|C| threshold from the whole reference, as the reference's
    own check takes it, reference bench.py:641-646); empty groups exactly zero."""
    offs = p.group_offs.cpu().numpy()
    L_all, R_all = p.lhs.cpu().numpy(), p.rhs.cpu().numpy()
    if p.is_mx:
        LS, RS = p.lhs_mx.cpu().numpy(), p.rhs_mx.cpu().numpy()
    got = pkg.as_bf16_bits(out)
    refs = []
    for g in range(p.G):
        lo, hi = int(offs[g]), int(offs[g + 1])
        sub = np.array([0, hi - lo], dtype=np.int64)
        if p.is_mx:
            b0, b1 = lo // 32, (hi + 31) // 32
            ref = orc.vark_wgrad_mxfp8(L_all[lo:hi], R_all[lo:hi], LS[b0:b1], RS[b0:b1], sub)[0]
        else:
            ref = orc.vark_wgrad_tensorwise(L_all[lo:hi], R_all[lo:hi], p.lhs_scale, p.rhs_scale, sub)[0]
        refs.append(ref)
        if hi == lo:
            assert np.all((got[g] & 0x7FFF) == 0), (p.name, "empty group", g)
    amax = max(float(np.abs(orc.bf16_bits_to_f32(r)).max()) for r in refs)
    m = orc.compare_parts(((got[g], refs[g]) for g in range(p.G)), amax)
    _say(f"{p.name}: whole C ({p.G} groups) vs oracle: {m}")
    assert orc.parity_ok(m), (p.name, m)


# one GPU's share of gate_up_wgrad sharded 8 ways without communication (bench.py's SHARD_CONFIGS)
SHARDS = {"gate_up_ep8": dict(G=4, M=65536), "gate_up_ncol8": dict(OUT_N=720), "gate_up_ncol6": dict(OUT_N=960)}


@pytest.mark.parametrize("name", ["down_wgrad", "gate_up_wgrad", "gate_up_zipf", "gate_up_mx", "gate_up_reference_lens",
                                  *SHARDS])
def test_full_size_config(pkg, orc, cuda, name):
    """Full-size configurations, the whole output against the oracle. gate_up_zipf and
    gate_up_reference_lens (the reference's seed-42 exponential group sizes) are skewed enough that
    the kernel deals its tiles in boustrophedon rounds rather than XCD-pair slices
    (tests/test_vark_schedule_host.py models the choice). gate_up_ep8 / gate_up_ncol8: one GPU's
    share under 8-way expert / N-column sharding (4 groups of ~16 K tokens; OUT_N = 720), and 6-way
    N-column sharding (OUT_N = 960)."""
    _say(f"full-size {name}")
    if name == "gate_up_reference_lens":
        p = pkg.inputs.make_problem("gate_up_wgrad", seed=0, device=cuda,
                                    lens=pkg.inputs.make_group_lens_reference())
    elif name in SHARDS:
        p = pkg.inputs.make_problem("gate_up_wgrad", seed=0, device=cuda, **SHARDS[name])
    else:
        p = pkg.inputs.make_problem(name, seed=0, device=cuda)
    if p.is_mx:
        run = lambda: pkg.grouped_gemm_mxfp8_variable_k(p.lhs, p.rhs, p.lhs_mx, p.rhs_mx, p.group_offs)
    else:
        sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=cuda)
        sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=cuda)
        run = lambda: pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs)
    out = run()
    out2 = run()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "non-deterministic output"
    assert bool(torch.isfinite(out).all())
    worst = _rowsum_identity(pkg, p, out, cuda)
    _say(f"{name}: row-sum identity worst relative residual {worst:.3e}")
    assert worst < 2 ** -6
    worst = _colsum_identity(pkg, p, out, cuda)
    _say(f"{name}: column-sum identity worst relative residual {worst:.3e}")
    assert worst < 2 ** -6
    _oracle_whole(pkg, orc, p, out)


# ----------------------------------------------------------------------------- fp32 epilogues

def _f32_parity(orc, got, ref, label):
    """The bar on fp32 values: cosine >= 0.99999, max relative error <= 2e-2 over |ref| >
    1e-3 max|ref|, all finite."""
    a = got.astype(np.float64).ravel()
    b = ref.astype(np.float64).ravel()
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
    mask = np.abs(b) > 1e-3 * np.abs(b).max()
    rel = float(np.max(np.abs(a[mask] - b[mask]) / np.abs(b[mask]))) if mask.any() else 0.0
    _say(f"{label}: cos {cos:.9f} max_rel {rel:.3e}")
    assert cos >= 0.99999 and rel <= 2e-2 and np.isfinite(a).all(), (label, cos, rel)


@pytest.mark.parametrize("lens,om,on", [([127, 128, 0, 255, 256, 257], 208, 336), ([300, 0, 645], 400, 1152),
                                        ([31] * 4 + [0] * 2, 16, 384)], ids=["c320", "c384", "tiny"])
def test_fp32_output_and_accumulate(pkg, orc, cuda, lens, om, on):
    lhs, rhs, offs, _, (sl, sr) = _rand_bytes_problem(lens, om, on, seed=len(lens) + om)
    G = len(lens)
    _say(f"fp32 out lens={lens} {om}x{on}")
    ref = orc.vark_wgrad_tensorwise_f32(lhs.numpy(), rhs.numpy(), sl, sr, offs.numpy(), acc_dtype=np.float64)
    dl, dr, do = lhs.to(cuda), rhs.to(cuda), offs.to(cuda)
    s1 = torch.tensor(sl, dtype=torch.float32, device=cuda)
    s2 = torch.tensor(sr, dtype=torch.float32, device=cuda)
    out = torch.full((G, om, on), float("nan"), dtype=torch.float32, device=cuda)
    pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, do, out=out, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    _f32_parity(orc, got, ref, "fp32 out")
    for g, L in enumerate(lens):
        if L == 0:
            assert np.all(got[g] == 0), g           # empty groups: exact zeros, NaN prefill overwritten
    # the fp32 result agrees with the bf16 kernel to bf16 rounding
    bf = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, do)
    assert torch.equal(out.to(torch.bfloat16).view(torch.int16), bf.view(torch.int16)) or \
        float((out.to(torch.bfloat16).float() - bf.float()).abs().max()) <= float(bf.float().abs().max()) * 2 ** -7
    # accumulate: C0 + result, twice in a row (C0 + 2 result)
    c0 = torch.randn((G, om, on), generator=torch.Generator().manual_seed(5)).float()
    acc = c0.to(cuda)
    pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, do, out=acc, accumulate=True)
    torch.cuda.synchronize()
    got1 = acc.cpu().numpy()
    _f32_parity(orc, got1 - c0.numpy(), ref, "accumulate once (minus C0)")
    _f32_parity(orc, got1, c0.numpy() + ref, "accumulate once")
    # the addition is the last rounding: C0 + fp32(result), exactly
    np.testing.assert_array_equal(got1, (c0.numpy() + got).astype(np.float32))
    pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, do, out=acc, accumulate=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), (got1 + got).astype(np.float32))


@pytest.mark.parametrize("routing", ["multinomial", "reference_lens"])
def test_fp32_accumulate_full_size(pkg, orc, cuda, routing):
    """gate_up_wgrad with fp32 main-grad accumulation: C0 + result equals the fp32-output run plus
    C0 exactly, on the whole 32 x 2880 x 5760 tensor, with uniform routing (the slices deal) and
    with the reference's exponential group sizes (the rounds deal, as in the layer step)."""
    _say(f"fp32 accumulate full-size gate_up ({routing})")
    lens = pkg.inputs.make_group_lens_reference() if routing == "reference_lens" else None
    p = pkg.inputs.make_problem("gate_up_wgrad", seed=0, device=cuda, lens=lens)
    sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=cuda)
    sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=cuda)
    f32 = pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs, out_dtype=torch.float32)
    c0 = torch.randn(f32.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(1)) * 1e-2
    acc = c0.clone()
    pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs, out=acc, accumulate=True)
    bf = pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs)
    torch.cuda.synchronize()
    assert torch.equal(acc, c0 + f32)
    assert torch.equal(f32.to(torch.bfloat16).view(torch.int16), bf.view(torch.int16))


# ----------------------------------------------------------------------------- launch contract

@pytest.mark.parametrize("kind", ["bf16", "f32", "f32_acc", "mx"])
def test_offsets_past_token_count_are_clamped(pkg, orc, cuda, kind):
    """Group offsets past M_total (the tensors' token count) are clamped on the device: lhs and
    rhs are views of the first M rows of larger buffers whose extra rows hold 0x38 (1.0 / 0.5), so
    any read past row M would change the result, which must equal the oracle on the clamped
    offsets (a negative first offset clamps to 0; a group wholly past M is empty)."""
    mx = kind == "mx"
    M = 448 if mx else 457
    offs = torch.tensor([0, 96, 96, 384, 640, 800] if mx else [-64, 100, 100, 400, 600, 800], dtype=torch.int64)
    clamped = offs.clamp(min=0, max=M)
    _say(f"wgrad offsets past M_total ({kind}): M={M} offs={offs.tolist()}")
    lens = torch.diff(clamped).tolist()
    lhs, rhs, _, sc, (sl, sr) = _rand_bytes_problem(lens, 208, 384, seed=41, mx=mx)
    pad = 512
    lhs_full = torch.cat([lhs, torch.full((pad, lhs.shape[1]), 0x38, dtype=torch.uint8)])
    rhs_full = torch.cat([rhs, torch.full((pad, rhs.shape[1]), 0x38, dtype=torch.uint8)])
    dl, dr = lhs_full.to(cuda)[:M], rhs_full.to(cuda)[:M]
    if mx:
        lsc = torch.cat([sc[0], torch.full((pad // 32, sc[0].shape[1]), 127, dtype=torch.uint8)])
        rsc = torch.cat([sc[1], torch.full((pad // 32, sc[1].shape[1]), 127, dtype=torch.uint8)])
        out = pkg.grouped_gemm_mxfp8_variable_k(dl, dr, lsc.to(cuda)[:M // 32], rsc.to(cuda)[:M // 32], offs.to(cuda))
        torch.cuda.synchronize()
        ref = orc.vark_wgrad_mxfp8(lhs.numpy(), rhs.numpy(), sc[0].numpy(), sc[1].numpy(), clamped.numpy())
        _assert_parity(orc, pkg.as_bf16_bits(out), ref, clamped.numpy(), "clamp/mx")
        return
    s1 = torch.tensor(sl, dtype=torch.float32, device=cuda)
    s2 = torch.tensor(sr, dtype=torch.float32, device=cuda)
    if kind == "bf16":
        out = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, offs.to(cuda))
        torch.cuda.synchronize()
        ref = orc.vark_wgrad_tensorwise(lhs.numpy(), rhs.numpy(), sl, sr, clamped.numpy())
        _assert_parity(orc, pkg.as_bf16_bits(out), ref, clamped.numpy(), "clamp/bf16")
        return
    c0 = torch.zeros((5, 208, 384), dtype=torch.float32, device=cuda)
    out = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, s1, s2, offs.to(cuda), out=c0,
                                                     out_dtype=torch.float32, accumulate=kind == "f32_acc")
    torch.cuda.synchronize()
    ref = orc.vark_wgrad_tensorwise_f32(lhs.numpy(), rhs.numpy(), sl, sr, clamped.numpy(), acc_dtype=np.float64)
    _f32_parity(orc, out.cpu().numpy(), ref, f"clamp/{kind}")
    for g in (1, 4):
        assert bool((out[g] == 0).all()), g


@pytest.mark.parametrize("dyn_lds", [32768, 0])
def test_code_object_short_dynamic_lds_writes_nan(pkg, cuda, dyn_lds):
    """A launch with less than the contracted 64 KiB of dynamic LDS computes nothing and fills
    C[0:G] with NaN (0x7FC0) instead of leaving it stale: the reference launcher never re-zeroes C
    between launches (launcher.cpp:108,163-169), so a mis-launch must not time as a valid run. A
    normal kernel exit, not a fault; a padded C shows nothing outside C[0:G] is written."""
    from ggemm_asm_amd import harness
    _say(f"wgrad code object with {dyn_lds} B dynamic LDS")
    lhs, rhs, offs, _, _ = _rand_bytes_problem([96, 0, 160], 192, 384, seed=23)
    dl, dr, do = lhs.to(cuda), rhs.to(cuda), offs.to(cuda)
    s = torch.tensor(0.1, device=cuda)
    big = torch.full((4, 200, 400), 0x1234, dtype=torch.int16, device=cuda)
    out = big.view(torch.bfloat16)[:3, :192, :384]
    module, func, _ = harness.load_kernel(pkg.CODE_OBJECT_PATH)
    try:
        harness.launch_variable_k_kernel(func, dl, dr, out, s, s, do, 3, 192, 384, harness.get_num_cus(0),
                                         shared_mem=dyn_lds)
        torch.cuda.synchronize()
    finally:
        harness.unload_kernel(module)
    assert bool((out.view(torch.int16) == 0x7FC0).all())
    big[:3, :192, :384] = 0x1234
    assert bool((big == 0x1234).all())
