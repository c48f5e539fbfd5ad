"""GPU parity of the FP8 quantization producer against the CPU oracle (launches through the C ABI).

Quantization is byte work: every fp8 byte, e8m0 byte, scale, amax and padded offset must equal
the oracle's exactly.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TDT = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _bytes(t):
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_amax(pkg, orq, cuda, dtype):
    g = torch.Generator().manual_seed(1)
    x = torch.randn((1000, 264), generator=g).to(dtype)
    x[517, 3] = -7.25                                   # the max is negative
    _say(f"amax {dtype}")
    a = pkg.amax(x.to(cuda))
    assert float(a) == float(orq.amax(x.float().numpy())) == 7.25
    x[2, 2] = float("nan")
    assert torch.isnan(pkg.amax(x.to(cuda))).item()
    z = torch.zeros((0, 64), dtype=dtype, device=cuda)
    assert float(pkg.amax(z)) == 0.0
    q, scale, am = pkg.quantize_fp8_tensorwise(z, "e4m3")
    assert q.shape == (0, 64) and float(scale) == 1.0 and float(am) == 0.0


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(4096, 2880), (777, 136), (3, 8)])
def test_tensorwise_bit_exact(pkg, orq, cuda, fmt, dtype, shape):
    g = torch.Generator().manual_seed(shape[0])
    x = (torch.randn(shape, generator=g) * (1e-3 if fmt == "e5m2" else 1.0)).to(dtype)
    _say(f"tensorwise {fmt} {dtype} {shape}")
    q, scale, am = pkg.quantize_fp8_tensorwise(x.to(cuda), fmt)
    torch.cuda.synchronize()
    q_ref, s_ref, a_ref = orq.quantize_tensorwise(x.float().numpy(), fmt)
    assert q.dtype == TDT[fmt] and q.shape == x.shape
    assert float(am) == float(a_ref) and float(scale) == float(s_ref)
    np.testing.assert_array_equal(_bytes(q), q_ref)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_tensorwise_rounding_ties_and_subnormals(pkg, orq, cuda, fmt):
    """amax = fmax makes the scale 1, so x / scale is exact and every fp8 tie, both fp32 neighbours
    of each tie, and fp32 subnormals reach the conversion unchanged."""
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(TDT[fmt]).float().numpy()
    vals = np.sort(np.unique(b[np.isfinite(b) & (b >= 0)]))
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    tiny = np.arange(1, 2000, dtype=np.uint32).view(np.float32)
    v = np.concatenate([vals, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)), tiny])
    v = np.concatenate([v, -v, [np.float32(orq.FMAX[fmt])], [-0.0]]).astype(np.float32)
    v = np.concatenate([v, np.zeros((-v.size) % 64, np.float32)]).reshape(-1, 64)
    _say(f"tensorwise ties {fmt} {v.shape}")
    q, scale, _ = pkg.quantize_fp8_tensorwise(torch.from_numpy(v).to(cuda), fmt)
    torch.cuda.synchronize()
    assert float(scale) == 1.0
    q_ref, _, _ = orq.quantize_tensorwise(v, fmt)
    np.testing.assert_array_equal(_bytes(q), q_ref)


def _near_tie_inputs(fmt, amax, seed):
    """fp32 inputs whose quotients x / scale lie within 4 fp32 ulps of every fp8 tie and value, for
    a scale that is not a power of two, plus random values up to amax, values small enough for the
    division's residual to underflow (|x| < 2^-102), amax itself and signed zeros."""
    scale = np.float32(np.float32(amax) / orq_fmax(fmt))
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(TDT[fmt]).float().numpy()
    vals = np.sort(np.unique(b[np.isfinite(b) & (b >= 0)]))
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    x0 = np.concatenate([vals[1:], mids]) * scale
    x = [x0.astype(np.float32)]
    up, dn = x[0].copy(), x[0].copy()
    for _ in range(4):
        up, dn = np.nextafter(up, np.float32(np.inf)), np.nextafter(dn, np.float32(0))
        x += [up, dn]
    rng = np.random.default_rng(seed)
    x.append((rng.uniform(-1, 1, 1 << 16) * np.float64(amax)).astype(np.float32))
    x.append(np.ldexp(np.float32(1.0), -np.arange(102, 150)).astype(np.float32))
    v = np.concatenate(x)
    v = v[np.abs(v) <= np.float32(amax)]
    v = np.concatenate([v, -v, [np.float32(amax), np.float32(-0.0), np.float32(0.0)]]).astype(np.float32)
    return np.concatenate([v, np.zeros((-v.size) % 1024, np.float32)]).reshape(-1, 64)   # rows: multiple of 16


def orq_fmax(fmt):
    return np.float32(448.0 if fmt == "e4m3" else 57344.0)


# amax values: ordinary non-power-of-two scales, the smallest amax (2^-60) the kernels' FMA-corrected
# quotient covers and one below it (the plain division), and one near the largest fp32
NEAR_TIE_AMAX = [613.76, 1.3e-4, 2.0 ** -60, 2.0 ** -61 * 1.7, 3.0e38]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("amax", NEAR_TIE_AMAX, ids=[f"a{i}" for i in range(len(NEAR_TIE_AMAX))])
def test_tensorwise_quotients_near_ties(pkg, orq, cuda, fmt, amax):
    """x / scale must be the correctly rounded fp32 quotient before the fp8 rounding: quotients a
    few ulps either side of each fp8 tie tell a faithful or double-rounded quotient from the correct
    one. Both producers (plain and transposing) against the oracle's bytes."""
    v = _near_tie_inputs(fmt, amax, seed=len(fmt))
    _say(f"tensorwise near ties {fmt} amax={amax} {v.shape}")
    q_ref, s_ref, a_ref = orq.quantize_tensorwise(v, fmt)
    assert float(a_ref) == np.float32(amax)
    q, scale, am = pkg.quantize_fp8_tensorwise(torch.from_numpy(v).to(cuda), fmt)
    torch.cuda.synchronize()
    assert float(am) == float(a_ref) and float(scale) == float(s_ref)
    np.testing.assert_array_equal(_bytes(q), q_ref)
    w = torch.from_numpy(v).reshape(1, -1, 64).to(cuda)
    q, q_t, scale, _ = pkg.quantize_fp8_tensorwise_transpose(w, fmt)
    torch.cuda.synchronize()
    assert float(scale) == float(s_ref)
    np.testing.assert_array_equal(_bytes(q).reshape(-1, 64), q_ref)
    np.testing.assert_array_equal(_bytes(q_t)[0], q_ref.T)


def _is_nan_code(b, fmt):
    """e4m3fn has one NaN code per sign (0x7F); in e5m2 every code with the exponent all ones and a
    nonzero mantissa (0x7D-0x7F) is a NaN."""
    return (b & 0x7F) == 0x7F if fmt == "e4m3" else (b & 0x7F) > 0x7C


def _assert_bytes_nan_signless(got, ref, fmt="e4m3"):
    """Bytes equal, except where the oracle's byte is a NaN code: there any NaN code of the format,
    with either sign, passes (the sign of a NaN result is unspecified, the GPU's x / NaN and numpy's
    differ there, and e5m2 has several NaN codes)."""
    nan = _is_nan_code(ref, fmt)
    assert np.all(_is_nan_code(got[nan], fmt))
    np.testing.assert_array_equal(got[~nan], ref[~nan])


def test_tensorwise_special_values(pkg, orq, cuda):
    x = torch.zeros((16, 64), dtype=torch.bfloat16)
    _say("tensorwise zeros / NaN")
    q, scale, am = pkg.quantize_fp8_tensorwise(x.to(cuda), "e4m3")
    assert float(scale) == 1.0 and float(am) == 0.0 and int(_bytes(q).max()) == 0
    x[3, 5] = float("nan")
    q, scale, am = pkg.quantize_fp8_tensorwise(x.to(cuda), "e4m3")
    q_ref, s_ref, a_ref = orq.quantize_tensorwise(x.float().numpy(), "e4m3")
    assert np.isnan(float(scale)) and np.isnan(float(am))
    _assert_bytes_nan_signless(_bytes(q), q_ref)
    # a NaN element among finite ones: only that element is NaN, the rest quantize normally
    x = torch.randn((16, 64)).to(torch.bfloat16)
    amax_finite = float(x.float().abs().max())
    q, scale, am = pkg.quantize_fp8_tensorwise(x.to(cuda), "e5m2")
    q_ref, s_ref, _ = orq.quantize_tensorwise(x.float().numpy(), "e5m2")
    assert float(am) == amax_finite and float(scale) == float(s_ref)
    np.testing.assert_array_equal(_bytes(q), q_ref)


def test_tensorwise_weight_3d_and_strided(pkg, orq, cuda):
    g = torch.Generator().manual_seed(7)
    w = torch.randn((4, 96, 160), generator=g).to(torch.bfloat16)
    _say("tensorwise 3-D weight")
    q, scale, _ = pkg.quantize_fp8_tensorwise(w.to(cuda), "e4m3")
    q_ref, s_ref, _ = orq.quantize_tensorwise(w.float().numpy().reshape(-1, 160), "e4m3")
    assert q.shape == w.shape and float(scale) == float(s_ref)
    np.testing.assert_array_equal(_bytes(q).reshape(-1, 160), q_ref)
    wide = torch.randn((300, 256), generator=g).to(torch.bfloat16).to(cuda)
    view = wide[:, 64:64 + 128]
    q, scale, _ = pkg.quantize_fp8_tensorwise(view, "e5m2")
    q_ref, s_ref, _ = orq.quantize_tensorwise(view.float().cpu().numpy(), "e5m2")
    np.testing.assert_array_equal(_bytes(q), q_ref)


TRANSPOSE_CASES = [((3, 80, 48), torch.bfloat16, "e4m3"), ((2, 64, 128), torch.float32, "e5m2"),
                   ((1, 144, 208), torch.float32, "e4m3"), ((112, 16), torch.bfloat16, "e5m2"),
                   ((5, 16, 1040), torch.bfloat16, "e4m3"), ((2, 272, 80), torch.bfloat16, "e5m2"),
                   ((1, 208, 64), torch.float32, "e4m3")]


@pytest.mark.parametrize("shape,dtype,fmt", TRANSPOSE_CASES, ids=[f"t{i}" for i in range(len(TRANSPOSE_CASES))])
def test_tensorwise_transpose_bit_exact(pkg, orq, cuda, shape, dtype, fmt):
    """q and q^T against the oracle's bytes: ragged edges of the 128-row x 64-column tiles (rows
    80, 144, 208 = 128 + 80, 272 = 2 * 128 + 16; columns 48, 80, 208, 1040 = 16 * 65), fp32 and bf16
    input, a 2-D input, both formats."""
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * (1e-3 if fmt == "e5m2" else 1.0)).to(dtype)
    _say(f"tensorwise transpose {fmt} {dtype} {shape}")
    q, q_t, scale, am = pkg.quantize_fp8_tensorwise_transpose(x.to(cuda), fmt)
    torch.cuda.synchronize()
    R, C = shape[-2:]
    q_ref, s_ref, a_ref = orq.quantize_tensorwise(x.float().numpy().reshape(-1, C), fmt)
    q_ref = q_ref.reshape(shape)
    assert float(am) == float(a_ref) and float(scale) == float(s_ref)
    assert q.shape == x.shape and q_t.shape == shape[:-2] + (C, R) and q_t.dtype == TDT[fmt]
    np.testing.assert_array_equal(_bytes(q), q_ref)
    np.testing.assert_array_equal(_bytes(q_t), np.swapaxes(q_ref, -1, -2))
    q2, q_t2, _, _ = pkg.quantize_fp8_tensorwise_transpose(x.to(cuda), fmt, keep=False)
    assert q2 is None
    np.testing.assert_array_equal(_bytes(q_t2), _bytes(q_t))


@pytest.mark.parametrize("shape", [(2, 80, 2880), (96, 160)])
def test_row_aligned_outputs(pkg, orq, cuda, shape):
    """row_align=128: the same bytes in views whose rows start on 128-byte lines (padded buffers),
    for the plain and the transposing producer."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(shape, generator=g).to(torch.bfloat16)
    _say(f"row-aligned producer {shape}")
    q_ref, _, _ = orq.quantize_tensorwise(x.float().numpy().reshape(-1, shape[-1]), "e4m3")
    q_ref = q_ref.reshape(shape)
    q, scale, _ = pkg.quantize_fp8_tensorwise(x.to(cuda), "e4m3", row_align=128)
    assert q.shape == x.shape and q.stride(-2) % 128 == 0 and q.stride(-2) >= shape[-1]
    np.testing.assert_array_equal(_bytes(q), q_ref)
    qa, qt, _, _ = pkg.quantize_fp8_tensorwise_transpose(x.to(cuda), "e4m3", row_align=128)
    torch.cuda.synchronize()
    assert qa.stride(-2) % 128 == 0 and qt.stride(-2) % 128 == 0
    np.testing.assert_array_equal(_bytes(qa), q_ref)
    np.testing.assert_array_equal(_bytes(qt), np.swapaxes(q_ref, -1, -2))


def test_tensorwise_transpose_full_weight(pkg, cuda):
    """The gate_up weight [32, 5760, 2880]: q equals the tensorwise kernel's bytes and q^T is
    their transpose (byte for byte); an empty batch writes only amax and scale."""
    g = torch.Generator(device=cuda).manual_seed(3)
    w = (torch.randn((32, 5760, 2880), generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    _say("tensorwise transpose [32, 5760, 2880]")
    q, q_t, scale, am = pkg.quantize_fp8_tensorwise_transpose(w, "e4m3")
    q0, s0, a0 = pkg.quantize_fp8_tensorwise(w, "e4m3")
    torch.cuda.synchronize()
    assert float(am) == float(a0) and float(scale) == float(s0)
    assert torch.equal(q.view(torch.uint8), q0.view(torch.uint8))
    assert torch.equal(q_t.view(torch.uint8), q0.view(torch.uint8).transpose(1, 2).contiguous())
    del w, q, q_t, q0
    z = torch.zeros((0, 64, 32), dtype=torch.bfloat16, device=cuda)
    q, q_t, scale, am = pkg.quantize_fp8_tensorwise_transpose(z, "e5m2")
    assert q.shape == (0, 64, 32) and q_t.shape == (0, 32, 64) and float(scale) == 1.0 and float(am) == 0.0


MX_CASES = [
    ([5, 0, 33, 64, 1, 100], 48),
    ([32, 32, 0, 31], 272),
    ([1000, 24, 0, 0, 77], 2880 // 5),
    ([0, 0, 7], 16),
    ([4096 + 13], 512),
]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("lens,N", MX_CASES, ids=[f"mx{i}" for i in range(len(MX_CASES))])
def test_mx_grouped_bit_exact(pkg, orq, cuda, fmt, dtype, lens, N):
    g = torch.Generator().manual_seed(sum(lens) + N)
    M = sum(lens)
    x = (torch.randn((M, N), generator=g) * (1e-3 if fmt == "e5m2" else 1.0)).to(dtype)
    if M > 40:
        x[:32, : N // 2] = 0                                # all-zero blocks
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    _say(f"mx {fmt} {dtype} lens={lens} N={N}")
    q, sc, pad = pkg.quantize_mxfp8_grouped(x.to(cuda), offs.to(cuda), fmt)
    torch.cuda.synchronize()
    q_ref, sc_ref, pad_ref = orq.quantize_mx_grouped(x.float().numpy(), offs.numpy(), fmt, out_rows=q.shape[0])
    pad = pad.cpu().numpy()
    np.testing.assert_array_equal(pad, pad_ref)
    P = int(pad[-1])
    np.testing.assert_array_equal(_bytes(q)[:P], q_ref[:P])
    np.testing.assert_array_equal(sc.cpu().numpy()[:P // 32], sc_ref[:P // 32])


@pytest.mark.parametrize("seed", range(8))
def test_random_producer_shapes_bit_exact(pkg, orq, cuda, seed):
    """Seeded random shapes through every producer entry point, byte for byte against the oracle:
    per-tensor (plain and row-aligned), per-tensor with the transposed copy, grouped MX (G 1-40,
    empty and one-row groups, any multiple of 16 columns), bf16 and fp32 inputs, both formats."""
    rng = np.random.default_rng(3000 + seed)
    fmt = "e4m3" if seed % 2 == 0 else "e5m2"
    dtype = torch.bfloat16 if seed % 4 < 2 else torch.float32
    G = int(rng.integers(1, 41))
    lens = np.where(rng.integers(0, 4, G) == 0, 0, rng.integers(1, 300, G))
    M, N = int(lens.sum()), 16 * int(rng.integers(1, 60))
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((M, N), generator=g) * float(10.0 ** rng.uniform(-4, 2))).to(dtype)
    _say(f"random producer seed={seed} {fmt} {dtype} G={G} M={M} N={N}")
    xd = x.to(cuda)
    q_ref, s_ref, a_ref = orq.quantize_tensorwise(x.float().numpy(), fmt)
    for align in (None, 128):
        q, scale, am = pkg.quantize_fp8_tensorwise(xd, fmt, row_align=align)
        torch.cuda.synchronize()
        assert float(am) == float(a_ref) and float(scale) == float(s_ref)
        np.testing.assert_array_equal(_bytes(q), q_ref)
    R = 16 * (M // 16)
    if R:
        q, q_t, _, _ = pkg.quantize_fp8_tensorwise_transpose(xd[:R].contiguous(), fmt, row_align=128)
        torch.cuda.synchronize()
        r_ref, _, _ = orq.quantize_tensorwise(x[:R].float().numpy(), fmt)
        np.testing.assert_array_equal(_bytes(q), r_ref)
        np.testing.assert_array_equal(_bytes(q_t), r_ref.T)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    q, sc, pad = pkg.quantize_mxfp8_grouped(xd, offs.to(cuda), fmt)
    torch.cuda.synchronize()
    mq, msc, mpad = orq.quantize_mx_grouped(x.float().numpy(), offs.numpy(), fmt, out_rows=q.shape[0])
    pad = pad.cpu().numpy()
    np.testing.assert_array_equal(pad, mpad)
    P = int(pad[-1])
    np.testing.assert_array_equal(_bytes(q)[:P], mq[:P])
    np.testing.assert_array_equal(sc.cpu().numpy()[:P // 32], msc[:P // 32])


def test_mx_invalid_offsets_write_nothing(pkg, cuda):
    """Offsets past the rows (which the host cannot see) make the kernel's own check skip all
    writes: the outputs keep their previous contents."""
    x = torch.randn((64, 32), dtype=torch.float32, device=cuda)
    _say("mx invalid offsets")
    from ggemm_asm_amd import _lib
    q = torch.full((64 + 31 * 2 + 31, 32), 0x55, dtype=torch.uint8, device=cuda)
    sc = torch.full((q.shape[0] // 32, 32), 0x66, dtype=torch.uint8, device=cuda)
    pad = torch.full((3,), -9, dtype=torch.int64, device=cuda)
    for bad in ([0, 40, 65], [0, 50, 40], [-1, 10, 20]):
        offs = torch.tensor(bad, dtype=torch.int64, device=cuda)
        rc = _lib.load().ggemm_quant_mxfp8_grouped(x.data_ptr(), 1, 64, 32, 32, offs.data_ptr(), 2, 0, q.data_ptr(),
                                                   32, q.shape[0], sc.data_ptr(), 32, pad.data_ptr(),
                                                   torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert bool((q == 0x55).all()) and bool((sc == 0x66).all()) and bool((pad == -9).all()), bad


def test_mx_producer_feeds_mx_wgrad(pkg, orc, orq, cuda):
    """End to end: the producer quantizes x and dy of ragged groups (padding them to 32-token
    blocks) and the MXFP8 wgrad consumes its output; the result matches the oracle wgrad of the
    producer's bytes."""
    lens = [100, 0, 257, 31, 64]
    OUT_M, OUT_N = 192, 384
    g = torch.Generator().manual_seed(11)
    M = sum(lens)
    x = torch.randn((M, OUT_M), generator=g).to(torch.bfloat16)
    dy = (torch.randn((M, OUT_N), generator=g) * 1e-3).to(torch.bfloat16)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    _say("mx producer -> mx wgrad")
    ql, sl, pad = pkg.quantize_mxfp8_grouped(x.to(cuda), offs, "e4m3")
    qr, sr, pad2 = pkg.quantize_mxfp8_grouped(dy.to(cuda), offs, "e5m2")
    assert torch.equal(pad, pad2)
    out = pkg.grouped_gemm_mxfp8_variable_k(ql, qr, sl, sr, pad, validate=True)
    torch.cuda.synchronize()
    P = int(pad[-1])
    ref = orc.vark_wgrad_mxfp8(_bytes(ql)[:P], _bytes(qr)[:P], sl.cpu().numpy()[:P // 32], sr.cpu().numpy()[:P // 32],
                               pad.cpu().numpy())
    m = orc.compare(pkg.as_bf16_bits(out), ref, pad.cpu().numpy())
    _say(f"mx end to end: {m}")
    assert orc.parity_ok(m) and m["empty_zero"]


def test_tensorwise_producer_feeds_persistent_gemm(pkg, orc, orp, cuda):
    """End to end: bf16 activations and weights quantized per tensor feed the forward GEMM."""
    lens, K, N = [300, 0, 77], 256, 384
    g = torch.Generator().manual_seed(12)
    M = sum(lens)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(cuda)
    w = (torch.randn((len(lens), N, K), generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    _say("tensorwise producer -> persistent fwd")
    qx, sx, _ = pkg.quantize_fp8_tensorwise(x, "e4m3")
    qw, sw, _ = pkg.quantize_fp8_tensorwise(w, "e4m3")
    out = pkg.grouped_gemm_fp8_tensorwise(qx, qw, sx, sw, offs)
    torch.cuda.synchronize()
    ref = orp.grouped_fp8(_bytes(qx), _bytes(qw), float(sx), float(sw), offs.cpu().numpy())
    m = orc.compare(pkg.as_bf16_bits(out), ref)
    _say(f"tensorwise end to end: {m}")
    assert orc.parity_ok(m)


def _delayed(pkg, x, hist, slot, fmt, cuda):
    h = torch.from_numpy(np.asarray(hist, np.float32).copy()).to(cuda)
    q, scale = pkg.quantize_fp8_tensorwise_delayed(torch.from_numpy(x).to(cuda) if isinstance(x, np.ndarray)
                                                   else x.to(cuda), h, slot, fmt)
    torch.cuda.synchronize()
    return q, float(scale), h.cpu().numpy()


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(4096, 2880), (777, 136), (3, 8)])
def test_delayed_bit_exact(pkg, orq, cuda, fmt, dtype, shape):
    """Delayed scaling against the oracle: bytes, the scale from the history's other entries, and
    the whole new history (max |x| at the slot, the rest untouched), for histories below x's range
    (saturation), at it and above it; the slot's old entry (the largest) is ignored."""
    g = torch.Generator().manual_seed(shape[0] + 1)
    x = (torch.randn(shape, generator=g) * (1e-3 if fmt == "e5m2" else 1.0)).to(dtype)
    xf = x.float().numpy()
    am = float(np.abs(xf).max())
    rng = np.random.default_rng(shape[1])
    for hs, slot in ((0.5, 0), (1.0, 7), (3.0, 15)):
        hist = (rng.uniform(0.3, 1.0, 16) * am * hs).astype(np.float32)
        hist[slot] = 1e30
        _say(f"delayed {fmt} {dtype} {shape} history x{hs} slot {slot}")
        q, scale, h2 = _delayed(pkg, x, hist, slot, fmt, cuda)
        q_ref, s_ref, h_ref = orq.quantize_tensorwise_delayed(xf, hist, slot, fmt)
        assert q.dtype == TDT[fmt] and q.shape == x.shape
        assert scale == float(s_ref)
        np.testing.assert_array_equal(h2, h_ref)
        np.testing.assert_array_equal(_bytes(q), q_ref)


# history amax values: ordinary scales, the ends of the FMA-corrected quotient's scale range
# [2^-80, 2^100] (as amax = scale * fmax) and one past each end (the plain division)
DELAYED_AMAX = [613.76, 1.3e-4, "lo", "lo-", "hi", "hi+"]


def _delayed_amax(tag, fmt):
    fmax = float(orq_fmax(fmt))
    return {"lo": 2.0 ** -80 * fmax, "lo-": 2.0 ** -81 * fmax * 1.3, "hi": 2.0 ** 100 * fmax,
            "hi+": 2.0 ** 101 * fmax * 1.1}.get(tag, tag)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("tag", DELAYED_AMAX, ids=[f"a{i}" for i in range(len(DELAYED_AMAX))])
def test_delayed_quotients_near_ties_and_saturation(pkg, orq, cuda, fmt, tag):
    """The given-scale quotient is the correctly rounded one near every fp8 tie (x up to the
    history's amax), and x far beyond it saturates, products overflowing fp32 included: the inputs
    of the near-tie test plus the same scaled by 1.5, 2 +- ulps (the kernel's 2 fmax guard), 2^20
    and up to FLT_MAX, and infinities."""
    amax = np.float32(_delayed_amax(tag, fmt))
    v = _near_tie_inputs(fmt, float(amax), seed=3).reshape(-1)
    big = [v * np.float32(1.5), v * np.float32(2.0)]
    big += [np.nextafter(big[1], np.float32(np.inf)), np.nextafter(big[1], np.float32(0))]
    with np.errstate(over="ignore"):
        big += [v * np.float32(2.0 ** 20), np.float32(3.4e38) * np.sign(v[:4096])]
    w = np.concatenate([v] + [b.astype(np.float32) for b in big] + [[np.inf, -np.inf]]).astype(np.float32)
    w = np.where(np.isfinite(w) | np.isinf(w), w, 0).astype(np.float32)
    w = np.concatenate([w, np.zeros((-w.size) % 1024, np.float32)]).reshape(-1, 64)
    hist = np.array([0.0, amax, amax * np.float32(0.25), 0.0], np.float32)
    _say(f"delayed near ties {fmt} amax={amax} {w.shape}")
    q, scale, h2 = _delayed(pkg, w, hist, 3, fmt, cuda)
    q_ref, s_ref, h_ref = orq.quantize_tensorwise_delayed(w, hist, 3, fmt)
    assert scale == float(s_ref) and np.isinf(h2[3])
    np.testing.assert_array_equal(h2, h_ref)
    np.testing.assert_array_equal(_bytes(q), q_ref)


def test_delayed_special_histories_and_inputs(pkg, orq, cuda):
    x = torch.randn((64, 128)).to(torch.bfloat16)
    xf = x.float().numpy()
    _say("delayed zero history / NaN history / NaN input / empty input")
    q, scale, h2 = _delayed(pkg, x, np.zeros(4, np.float32), 2, "e4m3", cuda)     # scale 1
    q_ref, s_ref, h_ref = orq.quantize_tensorwise_delayed(xf, np.zeros(4, np.float32), 2, "e4m3")
    assert scale == 1.0 == s_ref
    np.testing.assert_array_equal(h2, h_ref)
    np.testing.assert_array_equal(_bytes(q), q_ref)
    hist = np.array([1.0, np.nan, 2.0], np.float32)                             # NaN entry: NaN scale
    q, scale, h2 = _delayed(pkg, x, hist, 0, "e5m2", cuda)
    q_ref, _, h_ref = orq.quantize_tensorwise_delayed(xf, hist, 0, "e5m2")
    assert np.isnan(scale) and h2[0] == h_ref[0] and np.isnan(h2[1])
    _assert_bytes_nan_signless(_bytes(q), q_ref, "e5m2")
    y = x.clone()
    y[5, 9] = float("nan")                                                       # NaN input: NaN amax
    q, scale, h2 = _delayed(pkg, y, np.array([3.0, 9.0], np.float32), 1, "e4m3", cuda)
    q_ref, s_ref, _ = orq.quantize_tensorwise_delayed(y.float().numpy(), np.array([3.0, 9.0], np.float32), 1,
                                                      "e4m3")
    assert scale == float(s_ref) and h2[0] == 3.0 and np.isnan(h2[1])
    _assert_bytes_nan_signless(_bytes(q), q_ref)
    z = torch.zeros((0, 64), dtype=torch.bfloat16)                               # no rows: amax 0
    q, scale, h2 = _delayed(pkg, z, np.array([448.0, 5.0], np.float32), 1, "e4m3", cuda)
    assert q.shape == (0, 64) and scale == 1.0 and h2[1] == 0.0 and h2[0] == 448.0


def test_delayed_cycle_matches_oracle(pkg, orq, cuda):
    """Eight calls cycling the slot through a 4-entry history, the first one seeded by the
    current-scaling quantizer, with the input's range growing and shrinking: each call's bytes and
    scale against the oracle run over the same sequence, and the history in step."""
    rng = np.random.default_rng(4)
    xs = [(rng.standard_normal((512, 256)) * m).astype(np.float32) for m in (1, 2, 8, 0.5, 1, 4, 0.1, 1)]
    _say("delayed cycle of 8 calls, history 4")
    q0, _, am = pkg.quantize_fp8_tensorwise(torch.from_numpy(xs[0]).to(cuda), "e4m3")
    h = torch.zeros(4, dtype=torch.float32, device=cuda)
    h[:1].copy_(am.reshape(1))
    h_ref = np.zeros(4, np.float32)
    h_ref[0] = orq.amax(xs[0])
    for n in range(1, len(xs)):
        q, scale = pkg.quantize_fp8_tensorwise_delayed(torch.from_numpy(xs[n]).to(cuda), h, n % 4, "e4m3")
        q_ref, s_ref, h_ref = orq.quantize_tensorwise_delayed(xs[n], h_ref, n % 4, "e4m3")
        torch.cuda.synchronize()
        assert float(scale) == float(s_ref), n
        np.testing.assert_array_equal(h.cpu().numpy(), h_ref)
        np.testing.assert_array_equal(_bytes(q), q_ref)


def test_device_slot_cycle_matches_oracle(pkg, orq, cuda):
    """The device-slot entries (the slot advanced by the call on the device) over nine calls through
    a 3-entry history, three wraps, with the input's range growing and shrinking: each call's bytes
    and scale against the oracle at slot n % 3, the history in step and the device slot equal to
    n % 3 after call n. Plain and transposing quantizers; the transposing one starts from an
    out-of-range slot value (57), which restarts at 0."""
    rng = np.random.default_rng(9)
    mags = (1, 3, 0.25, 8, 1, 0.5, 2, 16, 0.1)
    xs = [(rng.standard_normal((384, 160)) * m).astype(np.float32) for m in mags]
    ws = [(rng.standard_normal((2, 96, 64)) * m * 0.05).astype(np.float32) for m in mags]
    _say("device-slot delayed cycle of 9 calls, history 3")
    h = torch.tensor([orq.amax(xs[0]) * 2, 0.0, 0.0], dtype=torch.float32, device=cuda)
    hw = torch.tensor([0.0, 0.0, orq.amax(ws[0])], dtype=torch.float32, device=cuda)
    h_ref, hw_ref = h.cpu().numpy(), hw.cpu().numpy()
    slot = torch.tensor([2], dtype=torch.int32, device=cuda)       # the previous call's slot
    slot_w = torch.tensor([57], dtype=torch.int32, device=cuda)
    for n in range(len(xs)):
        q, scale = pkg.quantize_fp8_tensorwise_delayed(torch.from_numpy(xs[n]).to(cuda), h, slot, "e5m2",
                                                       row_align=128)
        qw, qwt, sw = pkg.quantize_fp8_tensorwise_transpose_delayed(torch.from_numpy(ws[n]).to(cuda), hw, slot_w,
                                                                   "e4m3")
        q_ref, s_ref, h_ref = orq.quantize_tensorwise_delayed(xs[n], h_ref, n % 3, "e5m2")
        w_ref, sw_ref, hw_ref = orq.quantize_tensorwise_delayed(ws[n].reshape(-1, 64), hw_ref, n % 3, "e4m3")
        torch.cuda.synchronize()
        assert int(slot) == n % 3 and int(slot_w) == n % 3, n
        assert float(scale) == float(s_ref) and float(sw) == float(sw_ref), n
        np.testing.assert_array_equal(h.cpu().numpy(), h_ref)
        np.testing.assert_array_equal(hw.cpu().numpy(), hw_ref)
        np.testing.assert_array_equal(_bytes(q), q_ref)
        np.testing.assert_array_equal(_bytes(qw).reshape(-1, 64), w_ref)
        np.testing.assert_array_equal(_bytes(qwt), w_ref.reshape(2, 96, 64).transpose(0, 2, 1))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape,dtype,align", [((4, 96, 160), torch.bfloat16, None), ((3, 272, 144), torch.float32, 128),
                                               ((1, 5760 // 4, 2880 // 4), torch.bfloat16, 128)])
def test_transpose_delayed_bit_exact(pkg, orq, cuda, fmt, shape, dtype, align):
    """The transposing pass with delayed scaling: q, q^T (the same bytes transposed per matrix),
    the scale and the new history against the oracle, for histories below (saturation), at and
    above the tensor's range; keep=False writes only q^T."""
    g = torch.Generator().manual_seed(shape[1])
    w = (torch.randn(shape, generator=g) * (1e-3 if fmt == "e5m2" else 0.05)).to(dtype)
    wf = w.float().numpy()
    B, R, C = shape
    am = float(np.abs(wf).max())
    rng = np.random.default_rng(shape[2])
    for hs, slot, keep in ((0.5, 1, True), (1.0, 0, False), (2.0, 5, True)):
        hist = (rng.uniform(0.3, 1.0, 6) * am * hs).astype(np.float32)
        hist[slot] = 7e20
        _say(f"transpose delayed {fmt} {shape} {dtype} align={align} history x{hs} slot {slot} keep={keep}")
        h = torch.from_numpy(hist.copy()).to(cuda)
        q, q_t, scale = pkg.quantize_fp8_tensorwise_transpose_delayed(w.to(cuda), h, slot, fmt, keep=keep,
                                                                      row_align=align)
        torch.cuda.synchronize()
        q_ref, s_ref, h_ref = orq.quantize_tensorwise_delayed(wf.reshape(-1, C), hist, slot, fmt)
        q_ref = q_ref.reshape(B, R, C)
        assert float(scale) == float(s_ref)
        np.testing.assert_array_equal(h.cpu().numpy(), h_ref)
        np.testing.assert_array_equal(_bytes(q_t), q_ref.transpose(0, 2, 1))
        if keep:
            np.testing.assert_array_equal(_bytes(q), q_ref)
        else:
            assert q is None


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("tag", ["lo", "hi+", 613.76])
def test_transpose_delayed_near_ties_and_saturation(pkg, orq, cuda, fmt, tag):
    amax = np.float32(_delayed_amax(tag, fmt))
    v = _near_tie_inputs(fmt, float(amax), seed=5).reshape(-1)
    with np.errstate(over="ignore"):
        w = np.concatenate([v, v * np.float32(3.0), v * np.float32(2.0 ** 30), [np.inf, -np.inf]]).astype(np.float32)
    w = np.concatenate([w, np.zeros((-w.size) % 1024, np.float32)]).reshape(1, -1, 64)
    hist = np.array([amax, 0.0, amax * np.float32(0.5)], np.float32)
    _say(f"transpose delayed near ties {fmt} amax={amax} {w.shape}")
    h = torch.from_numpy(hist.copy()).to(cuda)
    q, q_t, scale = pkg.quantize_fp8_tensorwise_transpose_delayed(torch.from_numpy(w).to(cuda), h, 1, fmt)
    torch.cuda.synchronize()
    q_ref, s_ref, h_ref = orq.quantize_tensorwise_delayed(w.reshape(-1, 64), hist, 1, fmt)
    assert float(scale) == float(s_ref)
    np.testing.assert_array_equal(h.cpu().numpy(), h_ref)
    np.testing.assert_array_equal(_bytes(q).reshape(-1, 64), q_ref)
    np.testing.assert_array_equal(_bytes(q_t)[0], q_ref.T)


def test_transpose_delayed_empty_batch(pkg, cuda):
    h = torch.tensor([3.0, 448.0], device=cuda)
    _say("transpose delayed B=0")
    q, q_t, scale = pkg.quantize_fp8_tensorwise_transpose_delayed(torch.zeros((0, 32, 48), device=cuda), h, 0)
    torch.cuda.synchronize()
    assert q.shape == (0, 32, 48) and q_t.shape == (0, 48, 32)
    assert float(scale) == 1.0 and h.tolist() == [0.0, 448.0]
