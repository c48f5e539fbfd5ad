"""GPU parity of the persistent fwd/dgrad grouped FP8 GEMM against the CPU oracle (launches through
the C ABI or the drop-in code objects).

Bar (from the north-star statement, applied to this kernel): cosine >= 0.99999, max relative error
<= 2e-2 over |C| > 1e-3 * max|C|, no non-finite values. Small and ragged cases are compared in full
with the oracle; adversarial all-codes inputs against a rigorous error bound of the exact result;
the full-size call sites with the oracle on every row plus the size-independent row-sum identity
``out[r] @ 1 = s_a s_b A[r] (B[g]^T 1)`` on every row.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _run(pkg, a, b, fmt, offs, sa, sb, dev, **kw):
    adt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    return pkg.grouped_gemm_fp8_tensorwise(
        a.to(dev).view(adt), b.to(dev).view(torch.float8_e4m3fn), torch.tensor(sa, dtype=torch.float32, device=dev),
        torch.tensor(sb, dtype=torch.float32, device=dev), offs.to(dev), **kw)


def _parity(pkg, orc, got, ref_bits, label, rows=None):
    g = pkg.as_bf16_bits(got)
    if rows is not None:
        g = g[:rows]
        ref_bits = ref_bits[:rows]
    m = orc.compare(g, ref_bits)
    _say(f"{label}: {m}")
    assert orc.parity_ok(m), (label, m)
    return m


def _within_bound(orc, orp, got_bits, a, b, offs, fmt, sa, sb):
    """Boolean [M, N]: |got - exact| <= bf16 output rounding + the fp8 MFMA accumulation bound of
    the exact rational result (oracle.fp8_mfma_error_bound_rows) + fp32 rounding of the scales."""
    dec = orc.decode_e4m3 if fmt == "e4m3" else orc.decode_e5m2
    av = dec(a).astype(np.float64)
    bv = orc.decode_e4m3(b).astype(np.float64)
    exact = orp.grouped_fp8_f32(a, b, sa, sb, offs, fmt, acc_dtype=np.float64)
    scale = float(np.float32(sa)) * float(np.float32(sb))
    bound = orp.fp8_mfma_error_bound_rows(av, bv, offs, scale)
    mag = np.zeros_like(exact)
    for gi in range(offs.size - 1):
        mag[offs[gi]:offs[gi + 1]] = np.abs(av[offs[gi]:offs[gi + 1]]) @ np.abs(bv[gi]).T * scale
    got = orc.bf16_bits_to_f32(got_bits).astype(np.float64)
    lim = 2.0 ** -8 * np.abs(exact) + 1.01 * bound + 4 * 2.0 ** -24 * mag + 1e-38
    return np.abs(got - exact) <= lim, np.abs(got - exact) / lim


def _parity_small_k(pkg, orc, orp, got, p, label):
    """The bar's cosine and finiteness on every element; its 2e-2 relative bound on every element
    except those whose exact value is a heavy cancellation of much larger products, which must
    instead lie within the rigorous MFMA error bound (at small K a block-truncated sum can be a
    few percent of such a result)."""
    g = pkg.as_bf16_bits(got)
    ref = orp.grouped_fp8(p.a.numpy(), p.b.numpy(), p.a_scale, p.b_scale, p.group_offs.numpy(), p.a_format)
    m = orc.compare(g, ref)
    assert m["cos"] >= 0.99999 and m["nonfinite"] == 0, (label, m)
    a_, b_ = orc.bf16_bits_to_f32(g).astype(np.float64), orc.bf16_bits_to_f32(ref).astype(np.float64)
    big = np.abs(b_) > 1e-3 * np.abs(b_).max()
    rel_bad = big & (np.abs(a_ - b_) > 2e-2 * np.abs(b_))
    ok, ratio = _within_bound(orc, orp, g, p.a.numpy(), p.b.numpy(), p.group_offs.numpy(), p.a_format,
                              p.a_scale, p.b_scale)
    _say(f"{label}: {m}; {int(rel_bad.sum())} elements past 2e-2 relative, all within the MFMA bound: "
         f"{bool(ok[rel_bad].all())} (worst bound ratio overall {float(ratio.max()):.3f})")
    assert ok[rel_bad].all() and ok.all(), label


RAGGED = [
    # lens, K, N: 320-wide N tiles and 384-wide (N % 384 == 0, or N >= 1536 with the last tile at
    # least half full: 1728, 2880), partial M/N tiles, K tails
    ([1, 2, 3, 5, 8, 13, 21, 31], 128, 128),
    ([0, 0, 193, 0], 256, 384),
    ([191, 192, 193, 0, 385], 2880, 336),
    ([1000, 24], 208, 768),
    ([7], 16, 16),
    ([300, 0, 645], 5760, 640),
    ([64, 0, 96, 45], 144, 1152),
    ([383, 1], 2880, 2880),
    ([200, 77], 272, 1728),
]


@pytest.mark.parametrize("seed", range(10))
def test_random_shapes_vs_oracle(pkg, orc, orp, cuda, seed):
    """Seeded random configurations: G in 1..40 with empty, single-row, partial and multi-tile
    groups; K any multiple of 16 up to 1024 (K tails inside a stage), N any multiple of 16 up to
    800 or 1536 / 1728 / 1920 (both tile widths and the wide-tile rule); both A formats; the
    reference's value recipe. The bar on every row, or, where a heavy cancellation at small K
    exceeds its 2e-2 threshold, every element within the rigorous MFMA error bound."""
    rng = np.random.default_rng(2000 + seed)
    G = int(rng.integers(1, 41))
    kind = rng.integers(0, 4, G)
    lens = np.where(kind == 0, 0, np.where(kind == 1, rng.integers(1, 192, G), rng.integers(192, 700, G)))
    K = 16 * int(rng.integers(1, 65))
    N = 16 * int(rng.choice([int(rng.integers(1, 51)), 96, 108, 120]))
    fmt = "e4m3" if seed % 2 == 0 else "e5m2"
    site = "down_fwd" if fmt == "e4m3" else "down_dgrad"
    _say(f"persistent random seed={seed} G={G} M={int(lens.sum())} K={K} N={N} {fmt}")
    p = pkg.inputs.make_fwd_problem(site, seed=seed, lens=lens.tolist(), K=K, N=N)
    out = _run(pkg, p.a, p.b, fmt, p.group_offs, 0.1, 0.1, cuda)
    torch.cuda.synchronize()
    ref = orp.grouped_fp8(p.a.numpy(), p.b.numpy(), 0.1, 0.1, p.group_offs.numpy(), fmt)
    m = orc.compare(pkg.as_bf16_bits(out), ref)
    _say(f"random {seed}: {m}")
    if not orc.parity_ok(m):
        # at small K a heavy cancellation can pass 2e-2 relative; the rigorous bound cannot
        _parity_small_k(pkg, orc, orp, out, p, f"random {seed}")


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("lens,K,N", RAGGED, ids=[f"case{i}" for i in range(len(RAGGED))])
def test_ragged_vs_oracle(pkg, orc, orp, cuda, fmt, lens, K, N):
    site = "down_fwd" if fmt == "e4m3" else "down_dgrad"
    _say(f"persistent {fmt} lens={lens} K={K} N={N}")
    p = pkg.inputs.make_fwd_problem(site, seed=len(lens) + K, lens=lens, K=K, N=N)
    out = _run(pkg, p.a, p.b, fmt, p.group_offs, 0.1, 0.1, cuda)
    torch.cuda.synchronize()
    ref = orp.grouped_fp8(p.a.numpy(), p.b.numpy(), 0.1, 0.1, p.group_offs.numpy(), fmt)
    _parity(pkg, orc, out, ref, f"{fmt} {lens} K={K} N={N}", rows=int(sum(lens)))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_all_fp8_codes_error_bound(pkg, orc, orp, cuda, fmt):
    """Uniformly random finite codes over the whole exponent range: |got - exact| within bf16
    rounding plus the MFMA accumulation bound of the exact rational result."""
    lens, K, N = [100, 0, 333, 64], 400, 336
    g = torch.Generator().manual_seed(5)
    M = sum(lens)
    a = torch.randint(0, 256, (M, K), generator=g, dtype=torch.int32).to(torch.uint8)
    b = torch.randint(0, 256, (len(lens), N, K), generator=g, dtype=torch.int32).to(torch.uint8)
    if fmt == "e4m3":
        a[(a & 0x7F) == 0x7F] = 0x3A
    else:
        a[(a & 0x7C) == 0x7C] = 0x3B
    b[(b & 0x7F) == 0x7F] = 0x3A
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    sa, sb = 0.0173, 2.9e-4
    _say(f"persistent all-codes {fmt}")
    out = _run(pkg, a, b, fmt, offs, sa, sb, cuda)
    torch.cuda.synchronize()
    ok, ratio = _within_bound(orc, orp, pkg.as_bf16_bits(out), a.numpy(), b.numpy(), offs.numpy(), fmt, sa, sb)
    _say(f"{fmt}: violations {int((~ok).sum())} of {ok.size}, worst ratio {float(ratio.max()):.3f}")
    assert ok.all()


def test_rows_outside_groups_untouched_and_empty_input(pkg, orc, orp, cuda):
    lens, K, N = [50, 0, 200], 256, 384
    p = pkg.inputs.make_fwd_problem("gate_up_fwd", seed=3, lens=lens, K=K, N=N)
    M = p.M + 77                                   # 77 rows past offs[G]
    a = torch.cat([p.a, torch.full((77, K), 0x38, dtype=torch.uint8)])
    _say("persistent rows past offs[G] keep their contents")
    out = torch.full((M, N), -3.0, dtype=torch.bfloat16, device=cuda)
    res = pkg.grouped_gemm_fp8_tensorwise(
        a.to(cuda).view(torch.float8_e4m3fn), p.b.to(cuda).view(torch.float8_e4m3fn),
        torch.tensor(0.1, device=cuda), torch.tensor(0.1, device=cuda), p.group_offs.to(cuda), out=out)
    torch.cuda.synchronize()
    assert res.data_ptr() == out.data_ptr()
    assert bool((out[p.M:] == -3.0).all())
    ref = orp.grouped_fp8(a.numpy(), p.b.numpy(), 0.1, 0.1, p.group_offs.numpy())
    _parity(pkg, orc, out, ref, "rows past offs[G]", rows=p.M)
    # no rows at all: nothing is launched, the empty result comes back
    e = pkg.grouped_gemm_fp8_tensorwise(
        torch.empty((0, K), dtype=torch.float8_e4m3fn, device=cuda), p.b.to(cuda).view(torch.float8_e4m3fn),
        torch.tensor(0.1, device=cuda), torch.tensor(0.1, device=cuda),
        torch.zeros(len(lens) + 1, dtype=torch.int64, device=cuda))
    assert e.shape == (0, N)


@pytest.mark.parametrize("shape", [(3, 80, 48), (1, 144, 2880), (2, 272, 1040), (32, 2880, 5760)])
def test_transpose_u8(pkg, cuda, shape):
    """The byte transpose behind trans_b=False: every byte, ragged 128 x 128 edge tiles (rows 80,
    144, 272 = 2 * 128 + 16; columns 48, 1040 = 16 * 65), a strided source view, and the full
    gate_up weight in the [G, K, N] layout."""
    G, K, N = shape
    _say(f"byte transpose {shape}")
    g = torch.Generator(device=cuda).manual_seed(K + N)
    b = torch.randint(0, 256, (G, K, N), generator=g, device=cuda, dtype=torch.uint8)
    got = pkg.persistent.transpose_b(b.view(torch.float8_e4m3fn))
    assert got.shape == (G, N, K) and got.is_contiguous() and got.dtype == torch.float8_e4m3fn
    assert torch.equal(got.view(torch.uint8), b.transpose(1, 2).contiguous())
    if G * K * N < 1 << 24:
        wide = torch.randint(0, 256, (G, K + 5, N + 32), generator=g, device=cuda, dtype=torch.uint8)
        view = wide[:, 2:2 + K, 16:16 + N]
        assert torch.equal(pkg.persistent.transpose_b(view).view(torch.uint8), view.transpose(1, 2).contiguous())


def test_trans_b_false_and_strided_views(pkg, orc, orp, cuda):
    lens, K, N = [130, 70, 0, 260], 320, 400
    p = pkg.inputs.make_fwd_problem("down_dgrad", seed=4, lens=lens, K=K, N=N)
    ref = orp.grouped_fp8(p.a.numpy(), p.b.numpy(), 0.1, 0.1, p.group_offs.numpy(), "e5m2")
    s = torch.tensor(0.1, device=cuda)
    do = p.group_offs.to(cuda)
    _say("persistent trans_b=False")
    bt = p.b.to(cuda).view(torch.float8_e4m3fn).transpose(1, 2).contiguous()      # [G, K, N]
    out = pkg.grouped_gemm_fp8_tensorwise(p.a.to(cuda).view(torch.float8_e5m2), bt, s, s, do, trans_b=False)
    torch.cuda.synchronize()
    _parity(pkg, orc, out, ref, "trans_b=False")
    _say("persistent strided a / b / out")
    a_wide = torch.zeros((p.M, K + 64), dtype=torch.uint8, device=cuda)
    a_wide[:, 16:16 + K] = p.a.to(cuda)
    b_wide = torch.zeros((len(lens), N + 3, K + 32), dtype=torch.uint8, device=cuda)
    b_wide[:, :N, 32:] = p.b.to(cuda)
    o_wide = torch.zeros((p.M, N + 24), dtype=torch.bfloat16, device=cuda)
    av = a_wide[:, 16:16 + K].view(torch.float8_e5m2)
    bv = b_wide[:, :N, 32:].view(torch.float8_e4m3fn)
    assert av.stride(0) == K + 64 and bv.stride(1) == K + 32
    pkg.grouped_gemm_fp8_tensorwise(av, bv, s, s, do, out=o_wide[:, 8:8 + N])
    torch.cuda.synchronize()
    _parity(pkg, orc, o_wide[:, 8:8 + N], ref, "strided views")
    assert bool((o_wide[:, :8] == 0).all()) and bool((o_wide[:, 8 + N:] == 0).all())


@pytest.mark.parametrize("G", [300, 2047])
def test_many_groups(pkg, orc, orp, cuda, G):
    g = torch.Generator().manual_seed(G)
    lens = torch.randint(0, 40, (G,), generator=g)
    lens[torch.randint(0, G, (G // 3,), generator=g)] = 0
    lens[0] = 0
    lens[-1] = 5
    _say(f"persistent G={G} rows={int(lens.sum())}")
    p = pkg.inputs.make_fwd_problem("down_fwd", seed=G, lens=lens, K=48, N=32)
    out = _run(pkg, p.a, p.b, "e4m3", p.group_offs, 0.1, 0.1, cuda)
    torch.cuda.synchronize()
    _parity_small_k(pkg, orc, orp, out, p, f"G={G} K=48")


@pytest.mark.parametrize("fmt,N", [("e4m3", 768), ("e5m2", 640)])
def test_code_object_drop_in(pkg, cuda, fmt, N):
    """Our persistent .co launched like reference bench.py:312-361 (16-entry kernelParams, null
    stream, any grid) gives the library's result bit for bit."""
    from ggemm_asm_amd import harness
    lens, K = [96, 160, 0, 256, 33], 384
    p = pkg.inputs.make_fwd_problem("gate_up_fwd" if fmt == "e4m3" else "gate_up_dgrad", seed=21, lens=lens, K=K, N=N)
    adt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    da, db, do = p.a.to(cuda).view(adt), p.b.to(cuda).view(torch.float8_e4m3fn), p.group_offs.to(cuda)
    s1, s2 = torch.tensor(0.1, device=cuda), torch.tensor(0.1, device=cuda)
    _say(f"persistent code object {fmt} N={N}")
    ref = pkg.grouped_gemm_fp8_tensorwise(da, db, s1, s2, do)
    module, func, name = harness.load_kernel(pkg.PERSISTENT_CODE_OBJECT_PATHS[fmt])
    assert name == "_grouped_fp8_persistent_gemm_kernel"
    try:
        for grid in (harness.get_num_cus(0), 24, 20, 1):
            out = torch.zeros_like(ref)
            torch.cuda.synchronize()
            harness.launch_persistent_kernel(func, da, db, out, s1, s2, do, len(lens), N, K, grid)
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), grid
    finally:
        harness.unload_kernel(module)


# ----------------------------------------------------------------------------- full-size sites

def test_constant_fill_known_answer_full_size(pkg, cuda):
    """gate_up_fwd size, A bytes 0x38 (1.0), B bytes 0x40 (2.0), scales 0.1, K = 2880: every
    output is 0.01 * 2880 * 2 = 57.6, which is bf16 57.5 (0x4266)."""
    _say("persistent constant fill gate_up_fwd 131072x2880x5760")
    lens = pkg.inputs.make_group_lens_reference()
    offs = pkg.inputs.make_group_offs(lens).to(cuda)
    a = torch.full((131072, 2880), 0x38, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    b = torch.full((32, 5760, 2880), 0x40, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    s = torch.tensor(0.1, device=cuda)
    out = pkg.grouped_gemm_fp8_tensorwise(a, b, s, s, offs)
    torch.cuda.synchronize()
    assert bool((out.view(torch.int16) == 0x4266).all())


def _rowsum_identity(p, out, dev):
    """max over rows of |sum_n out - s_a s_b A[r] . (sum_n B[g, n, :])| / (sum_n |out| + eps)."""
    offs = p.group_offs.cpu().tolist()
    worst = 0.0
    adt = p.a_dtype
    for g in range(p.G):
        lo, hi = offs[g], offs[g + 1]
        if hi == lo:
            continue
        c = out[lo:hi].float()
        lhs = c.sum(dim=1).double()
        A = p.a[lo:hi].view(adt).double()
        colsum = p.b[g].view(torch.float8_e4m3fn).double().sum(dim=0)
        rhs = (A @ colsum) * float(np.float32(p.a_scale)) * float(np.float32(p.b_scale))
        worst = max(worst, float(((lhs - rhs).abs() / (c.abs().sum(dim=1).double() + 1e-30)).max()))
    return worst


@pytest.mark.parametrize("name", ["gate_up_fwd", "down_fwd", "down_dgrad", "gate_up_dgrad"])
def test_full_size_site(pkg, orc, orp, cuda, name):
    _say(f"persistent full-size {name}")
    p = pkg.inputs.make_fwd_problem(name, seed=0, device=cuda)
    sa = torch.tensor(p.a_scale, dtype=torch.float32, device=cuda)
    sb = torch.tensor(p.b_scale, dtype=torch.float32, device=cuda)
    run = lambda: pkg.grouped_gemm_fp8_tensorwise(p.a.view(p.a_dtype), p.b.view(torch.float8_e4m3fn), sa, sb,
                                                  p.group_offs)
    out = run()
    out2 = run()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "non-deterministic output"
    assert bool(torch.isfinite(out).all())
    worst = _rowsum_identity(p, out, cuda)
    _say(f"{name}: row-sum identity worst relative residual {worst:.3e}")
    assert worst < 2 ** -6
    # every row of every group against the oracle, the bar over the whole output
    offs = p.group_offs.cpu().numpy()
    a_all, b_all = p.a.cpu().numpy(), p.b.cpu().numpy()
    got = pkg.as_bf16_bits(out)
    refs = []
    for g in range(p.G):
        lo, hi = int(offs[g]), int(offs[g + 1])
        refs.append(orp.grouped_fp8(a_all[lo:hi], b_all[g:g + 1], p.a_scale, p.b_scale,
                                    np.array([0, hi - lo]), p.a_format))
    amax = max(float(np.abs(orc.bf16_bits_to_f32(r)).max()) if r.size else 0.0 for r in refs)
    m = orc.compare_parts(((got[offs[g]:offs[g + 1]], refs[g]) for g in range(p.G)), amax)
    _say(f"{name}: all {int(offs[-1])} rows vs oracle: {m}")
    assert orc.parity_ok(m), (name, m)


def test_offsets_past_row_count_are_clamped(pkg, orc, orp, cuda):
    """Group offsets past M_total (the rows of a and out) are clamped on the device: a and out are
    views of the first M rows of larger buffers whose extra rows hold 0x38 (A) and a sentinel
    (out); no row past M may be read (it would change the result) or written (the sentinel stays),
    and the rows within M equal the oracle on the clamped offsets. zero_tail clears the rows past
    the clamped offs[G] and only those."""
    M, K, N = 457, 272, 384
    offs = torch.tensor([0, 100, 100, 400, 600, 800], dtype=torch.int64)
    clamped = offs.clamp(max=M).numpy()
    _say(f"persistent offsets past M_total: M={M} offs={offs.tolist()}")
    g = torch.Generator().manual_seed(31)
    a_full = torch.full((M + 512, K), 0x38, dtype=torch.uint8)
    a_full[:M] = torch.randn((M, K), generator=g).to(torch.float8_e4m3fn).view(torch.uint8)
    b = torch.randn((5, N, K), generator=g).to(torch.float8_e4m3fn).view(torch.uint8)
    da = a_full.to(cuda)[:M].view(torch.float8_e4m3fn)
    s = torch.tensor(0.25, device=cuda)
    for zero_tail in (False, True):
        out_full = torch.full((M + 512, N), 0x1234, dtype=torch.int16, device=cuda)
        out = out_full.view(torch.bfloat16)[:M]
        pkg.grouped_gemm_fp8_tensorwise(da, b.to(cuda).view(torch.float8_e4m3fn), s, s, offs.to(cuda), out=out,
                                        zero_tail=zero_tail)
        torch.cuda.synchronize()
        assert bool((out_full[M:] == 0x1234).all()), "a row past M_total was written"
        ref = orp.grouped_fp8(a_full[:M].numpy(), b.numpy(), 0.25, 0.25, clamped, "e4m3")
        m = orc.compare(pkg.as_bf16_bits(out)[:int(clamped[-1])], ref[:int(clamped[-1])])
        _say(f"zero_tail={zero_tail}: {m}")
        assert orc.parity_ok(m)


def test_code_object_short_dynamic_lds_writes_nan(pkg, cuda):
    """A launch with less than the contracted 64 KiB of dynamic LDS computes nothing and fills the
    rows a valid launch writes, [0, offs[G]), with NaN (0x7FC0), so the mistake cannot pass for a
    fast valid run; rows past offs[G] stay untouched. A normal kernel exit, not a fault."""
    from ggemm_asm_amd import harness
    M, K, N = 300, 256, 384
    offs = torch.tensor([0, 120, 120, 250], dtype=torch.int64, device=cuda)
    a = torch.zeros((M, K), dtype=torch.uint8, device=cuda)
    b = torch.zeros((3, N, K), dtype=torch.uint8, device=cuda)
    s = torch.tensor(1.0, device=cuda)
    _say("persistent code object with 32 KiB dynamic LDS")
    module, func, _ = harness.load_kernel(pkg.PERSISTENT_CODE_OBJECT_PATHS["e4m3"])
    try:
        out = torch.full((M, N), 0x1234, dtype=torch.int16, device=cuda)
        harness.launch_persistent_kernel(func, a, b, out, s, s, offs, 3, N, K, harness.get_num_cus(0),
                                         shared_mem=32768)
        torch.cuda.synchronize()
    finally:
        harness.unload_kernel(module)
    assert bool((out[:250] == 0x7FC0).all())
    assert bool((out[250:] == 0x1234).all())
