"""CPU checks of the quantization producer: its C ABI (no kernel launches: every call here fails
validation, or passes it with nothing to launch, before any HIP call), and a model of the
transposing kernels' tile arithmetic (bounds, coverage, padding untouched) run before any GPU
launch of a new shape class."""
import os
import re

import numpy as np

import pytest
import torch

from conftest import ROOT

FAKE = 0x100000


def test_quant_header_symbols_exported(pkg):
    text = open(os.path.join(ROOT, "include", "ggemm_quant.h")).read()
    names = sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ggemm_quant_\w+)\s*\(", text, re.M)))
    from ggemm_asm_amd import _lib
    assert names == sorted(_lib.QUANT_EXPORTS)
    lib = pkg.load_library()
    for n in names:
        assert hasattr(lib, n)


def _tw(lib, **kw):
    a = dict(x=FAKE, dt=0, rows=100, cols=64, stride=64, fmt=0, out=FAKE, ostride=64, scale=FAKE, amax=FAKE)
    a.update(kw)
    return lib.ggemm_quant_fp8_tensorwise(a["x"], a["dt"], a["rows"], a["cols"], a["stride"], a["fmt"], a["out"],
                                          a["ostride"], a["scale"], a["amax"], None)


@pytest.mark.parametrize("kw,rc", [
    (dict(x=0), -1), (dict(out=0), -1), (dict(scale=0), -1), (dict(dt=2), -8), (dict(fmt=3), -8),
    (dict(cols=60, stride=64), -2), (dict(rows=-1), -2), (dict(stride=56), -3), (dict(stride=68), -3),
    (dict(ostride=60), -3), (dict(x=FAKE + 8), -4), (dict(out=FAKE + 4), -4),
])
def test_tensorwise_validation(pkg, kw, rc):
    assert _tw(pkg.load_library(), **kw) == rc


def _dl(lib, **kw):
    a = dict(x=FAKE, dt=0, rows=100, cols=64, stride=64, fmt=0, out=FAKE, ostride=64, hist=FAKE, H=16, slot=3,
             scale=FAKE)
    a.update(kw)
    return lib.ggemm_quant_fp8_tensorwise_delayed(a["x"], a["dt"], a["rows"], a["cols"], a["stride"], a["fmt"],
                                                  a["out"], a["ostride"], a["hist"], a["H"], a["slot"], a["scale"],
                                                  None)


@pytest.mark.parametrize("kw,rc", [
    (dict(x=0), -1), (dict(out=0), -1), (dict(hist=0), -1), (dict(scale=0), -1), (dict(dt=2), -8),
    (dict(fmt=3), -8), (dict(cols=60, stride=64), -2), (dict(rows=-1), -2), (dict(stride=56), -3),
    (dict(ostride=60), -3), (dict(H=0, slot=0), -2), (dict(H=1025), -2), (dict(slot=-1), -2),
    (dict(slot=16), -2), (dict(x=FAKE + 8), -4), (dict(out=FAKE + 4), -4), (dict(hist=FAKE + 2), -4),
    (dict(scale=FAKE + 1), -4),
])
def test_delayed_validation(pkg, kw, rc):
    assert _dl(pkg.load_library(), **kw) == rc


def _tdl(lib, **kw):
    a = dict(x=FAKE, dt=0, B=2, R=64, C=48, fmt=0, out=FAKE, os=48, out_t=FAKE, ts=64, hist=FAKE, H=16, slot=3,
             scale=FAKE)
    a.update(kw)
    return lib.ggemm_quant_fp8_tensorwise_transpose_delayed(a["x"], a["dt"], a["B"], a["R"], a["C"], a["fmt"],
                                                            a["out"], a["os"], a["out_t"], a["ts"], a["hist"], a["H"],
                                                            a["slot"], a["scale"], None)


@pytest.mark.parametrize("kw,rc", [
    (dict(x=0), -1), (dict(out_t=0), -1), (dict(hist=0), -1), (dict(scale=0), -1), (dict(dt=2), -8),
    (dict(fmt=2), -8), (dict(B=-1), -2), (dict(R=0), -2), (dict(C=40), -2), (dict(H=0, slot=0), -2),
    (dict(H=1025), -2), (dict(slot=-1), -2), (dict(slot=16), -2), (dict(x=FAKE + 8), -4),
    (dict(out_t=FAKE + 8), -4), (dict(hist=FAKE + 2), -4), (dict(os=32), -3), (dict(ts=48), -3),
])
def test_transpose_delayed_validation(pkg, kw, rc):
    assert _tdl(pkg.load_library(), **kw) == rc


def _dl_dev(lib, **kw):
    a = dict(x=FAKE, dt=0, rows=100, cols=64, stride=64, fmt=0, out=FAKE, ostride=64, hist=FAKE, H=16, slot=FAKE,
             scale=FAKE)
    a.update(kw)
    return lib.ggemm_quant_fp8_tensorwise_delayed_dev(a["x"], a["dt"], a["rows"], a["cols"], a["stride"], a["fmt"],
                                                      a["out"], a["ostride"], a["hist"], a["H"], a["slot"],
                                                      a["scale"], None)


def _tdl_dev(lib, **kw):
    a = dict(x=FAKE, dt=0, B=2, R=64, C=48, fmt=0, out=FAKE, os=48, out_t=FAKE, ts=64, hist=FAKE, H=16, slot=FAKE,
             scale=FAKE)
    a.update(kw)
    return lib.ggemm_quant_fp8_tensorwise_transpose_delayed_dev(a["x"], a["dt"], a["B"], a["R"], a["C"], a["fmt"],
                                                                a["out"], a["os"], a["out_t"], a["ts"], a["hist"],
                                                                a["H"], a["slot"], a["scale"], None)


@pytest.mark.parametrize("kw,rc", [
    (dict(slot=0), -1), (dict(hist=0), -1), (dict(x=0), -1), (dict(H=0), -2), (dict(H=1025), -2),
    (dict(slot=FAKE + 2), -4), (dict(hist=FAKE + 2), -4), (dict(fmt=3), -8), (dict(stride=56), -3),
])
def test_device_slot_delayed_validation(pkg, kw, rc):
    """The device-slot entries take any slot value (the kernel wraps it into [0, H)), but a null or
    misaligned slot pointer and the host-slot entries' other checks fail before any launch."""
    lib = pkg.load_library()
    assert _dl_dev(lib, **kw) == rc
    tkw = {k: v for k, v in kw.items() if k != "stride"}
    if tkw:
        assert _tdl_dev(lib, **tkw) == (-8 if tkw.get("fmt") == 3 else rc)


def test_delayed_python_checks_history(pkg):
    x = torch.zeros((16, 64))
    with pytest.raises(ValueError, match="GPU only"):
        pkg.quantize_fp8_tensorwise_delayed(x, torch.zeros(4), 0)
    from ggemm_asm_amd import autograd, quant
    with pytest.raises(ValueError, match="history_len"):
        autograd.FP8DelayedScaling(1)
    with pytest.raises(ValueError, match="one-element int32"):
        quant._check_history(torch.zeros(4), torch.zeros(1, dtype=torch.int64), torch.device("cpu"))
    with pytest.raises(ValueError, match="one-element int32"):
        quant._check_history(torch.zeros(4), torch.zeros(2, dtype=torch.int32), torch.device("cpu"))
    quant._check_history(torch.zeros(4), torch.zeros(1, dtype=torch.int32), torch.device("cpu"))


def _mx(lib, **kw):
    a = dict(x=FAKE, dt=0, rows=100, cols=64, stride=64, offs=FAKE, G=4, fmt=1, out=FAKE, ostride=64, orows=100 + 124,
             sc=FAKE, sstride=64, pad=FAKE)
    a.update(kw)
    return lib.ggemm_quant_mxfp8_grouped(a["x"], a["dt"], a["rows"], a["cols"], a["stride"], a["offs"], a["G"],
                                         a["fmt"], a["out"], a["ostride"], a["orows"], a["sc"], a["sstride"],
                                         a["pad"], None)


@pytest.mark.parametrize("kw,rc", [
    (dict(offs=0), -1), (dict(pad=0), -1), (dict(fmt=2), -8), (dict(G=0), -2), (dict(G=2048), -2),
    (dict(cols=72, stride=72, ostride=80, sstride=80), -2), (dict(orows=100 + 123), -2),
    (dict(rows=(1 << 31) - 100), -2), (dict(ostride=72), -3), (dict(sstride=48), -3),
    (dict(out=FAKE + 8), -4), (dict(sc=FAKE + 8), -4), (dict(offs=FAKE + 4), -4),
])
def test_mx_validation(pkg, kw, rc):
    assert _mx(pkg.load_library(), **kw) == rc


def _tt(lib, **kw):
    a = dict(x=FAKE, dt=0, B=2, R=64, C=48, fmt=0, out=FAKE, os=48, out_t=FAKE, ts=64, scale=FAKE, amax=FAKE)
    a.update(kw)
    return lib.ggemm_quant_fp8_tensorwise_transpose(a["x"], a["dt"], a["B"], a["R"], a["C"], a["fmt"], a["out"],
                                                    a["os"], a["out_t"], a["ts"], a["scale"], a["amax"], None)


@pytest.mark.parametrize("kw,rc", [
    (dict(x=0), -1), (dict(out_t=0), -1), (dict(scale=0), -1), (dict(amax=0), -1), (dict(dt=2), -8),
    (dict(fmt=2), -8), (dict(B=-1), -2), (dict(R=0), -2), (dict(C=40), -2), (dict(R=72), -2),
    (dict(x=FAKE + 8), -4), (dict(out=FAKE + 8), -4), (dict(out_t=FAKE + 8), -4), (dict(amax=FAKE + 2), -4),
    (dict(os=32), -3), (dict(os=56), -3), (dict(ts=48), -3), (dict(ts=72), -3),
])
def test_transpose_validation(pkg, kw, rc):
    assert _tt(pkg.load_library(), **kw) == rc


def test_python_quant_refuses_cpu_and_bad_dtypes(pkg):
    x = torch.zeros(8, 16)
    with pytest.raises(ValueError, match="gfx950 GPU only"):
        pkg.quantize_fp8_tensorwise(x)
    with pytest.raises(TypeError):
        pkg.quantize_fp8_tensorwise(x.half())
    with pytest.raises(ValueError, match="e4m3"):
        pkg.quantize_fp8_tensorwise(x, "e3m4")
    assert pkg.padded_rows(100, 4) == 224 and pkg.padded_rows(0, 1) == 32
    with pytest.raises(ValueError, match="gfx950 GPU only"):
        pkg.quantize_fp8_tensorwise_transpose(torch.zeros(2, 16, 32))


def test_grouped_linear_refuses_cpu(pkg):
    x = torch.zeros(8, 16, dtype=torch.bfloat16, requires_grad=True)
    w = torch.zeros(2, 32, 16, dtype=torch.bfloat16, requires_grad=True)
    offs = torch.tensor([0, 3, 8])
    with pytest.raises(ValueError, match="gfx950 GPU only"):
        pkg.grouped_linear_fp8(x, w, offs)
    with pytest.raises(ValueError, match="main_grad"):
        pkg.grouped_linear_fp8(x, w, offs, main_grad=torch.zeros(2, 32, 16))


# ----------------------------------------------------------------------------- transpose index model

def _tt_off(r, c):
    """quant_kernel.h's LDS tile map: 128-byte rows, 16-byte chunk k of row r at k ^ ((r >> 4) & 7)."""
    return r * 128 + ((((c >> 4) ^ (r >> 4)) & 7) << 4) + (c & 15)


def _transpose_model(B, R, C, q_stride, t_stride):
    """Restatement of the 128 x 128 tile arithmetic of quant_transpose_kernel and of
    ggemm_persistent_transpose_u8, which shares it (LDS map _tt_off, the transposed copy from the
    dwords of 4 columns x 16 rows per thread): every byte of q and of q^T written exactly once from
    the right source element, no access outside the buffers, and every q^T store instruction of a
    wave writing whole 128-byte segments."""
    T = P = 128
    loc = _tt_off
    rt, ct = -(-R // T), -(-C // T)
    per = rt * ct
    x = np.arange(B * R * C, dtype=np.int64).reshape(B, R, C)
    q = np.full(B * R * q_stride, -1, np.int64)
    qt = np.full(B * C * t_stride, -1, np.int64)
    for it in range(B * per):
        b, rem = divmod(it, per)
        r0, c0 = (rem // ct) * T, (rem % ct) * T
        lds = np.full(T * P, -1, np.int64)
        for tid in range(256):
            tr, tc = tid >> 3, 16 * (tid & 7)
            for h in range(4):
                if c0 + tc < C and r0 + tr + 32 * h < R:
                    row = b * R + r0 + tr + 32 * h
                    assert c0 + tc + 16 <= C
                    vals = x.reshape(-1)[row * C + c0 + tc: row * C + c0 + tc + 16]
                    o = row * q_stride + c0 + tc
                    assert o + 16 <= q.size and (q[o:o + 16] == -1).all()
                    q[o:o + 16] = vals
                    lo = loc(tr + 32 * h, tc)
                    assert lo + 16 <= T * P and all(loc(tr + 32 * h, tc + i) == lo + i for i in range(16))
                    lds[lo:lo + 16] = vals
        for k in range(4):                       # one store instruction per k
            for wave in range(4):
                segs = {}
                for lane in range(64):
                    tid = 64 * wave + lane
                    cg, rj = tid >> 3, tid & 7
                    if not (r0 + 16 * rj < R and c0 + 4 * cg < C):
                        continue
                    assert c0 + 4 * cg + 4 <= C and r0 + 16 * rj + 16 <= R
                    # dwords of columns 4 cg .. 4 cg + 3 of rows 16 rj + i, byte k of each
                    vals = []
                    for i in range(16):
                        d0 = _tt_off(16 * rj + i, 4 * cg)
                        assert d0 % 4 == 0 and all(_tt_off(16 * rj + i, 4 * cg + m) == d0 + m for m in range(4))
                        vals.append(lds[d0 + k])
                    assert min(vals) >= 0
                    o = (b * C + c0 + 4 * cg + k) * t_stride + r0 + 16 * rj
                    assert o + 16 <= qt.size and (qt[o:o + 16] == -1).all()
                    qt[o:o + 16] = vals
                    segs.setdefault(o - 16 * rj, []).append(rj)
                # 8 threads per q^T row: the 128 bytes from r0 (whole lines when t_stride and r0 are)
                assert all(sorted(v) == list(range(len(v))) for v in segs.values())
    qv = q.reshape(B, R, q_stride)[:, :, :C]
    tv = qt.reshape(B, C, t_stride)[:, :, :R]
    assert np.array_equal(qv, x) and np.array_equal(tv, np.swapaxes(x, 1, 2))
    # padding bytes are never written
    assert (q.reshape(B, R, q_stride)[:, :, C:] == -1).all() and (qt.reshape(B, C, t_stride)[:, :, R:] == -1).all()


@pytest.mark.parametrize("B,R,C,qs,ts", [
    (3, 80, 48, 48, 80), (1, 144, 208, 256, 256), (2, 272, 80, 128, 384), (1, 208, 64, 64, 208),
    (5, 16, 1040, 1040, 16), (1, 256, 384, 384, 256), (2, 16, 16, 128, 128),
])
def test_transpose_tile_index_model(B, R, C, qs, ts):
    _transpose_model(B, R, C, qs, ts)


def test_transpose_gather_conflict_free():
    """quant_transpose_kernel's LDS traffic: a wave's 16-byte row-chunk writes cover each 128-byte
    row once per 8 lanes, and each dword read instruction of the gather touches 16 distinct
    dwords in at most 2 passes of 32 banks (256 bytes for 64 lanes at 128 bytes per cycle)."""
    for wave in range(4):
        for h in range(4):
            addrs = [_tt_off((64 * wave + l >> 3) + 32 * h, 16 * (l & 7)) for l in range(64)]
            for g in range(8):
                banks = sorted((a // 4 + m) % 32 for a in addrs[8 * g:8 * g + 8] for m in range(4))
                assert banks == list(range(32))
        for i in range(16):
            dws = [_tt_off(16 * ((64 * wave + l) & 7) + i, 4 * ((64 * wave + l) >> 3)) // 4 for l in range(64)]
            per_bank = {}
            for dw in set(dws):
                per_bank.setdefault(dw % 32, set()).add(dw)
            assert max(len(v) for v in per_bank.values()) <= 2


def test_overlapping_rows_are_copied_not_read_past():
    """An input whose rows overlap (an expanded view: stride 0) is copied before the library sees
    it, and the row stride handed to the library is the tensor's own -- never a stride the view
    does not have (the kernels read rows * cols distinct elements); a view of one row passes its
    width (its stride(0) is arbitrary and unused)."""
    import torch
    from ggemm_asm_amd import quant
    x = torch.randn(1, 256).expand(1024, 256)
    x2 = quant._as_2d(x)
    assert x2.is_contiguous() and x2.stride(0) == 256 and torch.equal(x2, x)
    assert quant._row_stride(x2) == 256
    y = torch.randn(64, 512)[:, :256]                  # padded rows: the stride is kept
    assert quant._row_stride(quant._as_2d(y)) == 512
    z = torch.randn(300, 1, 256).expand(300, 2, 256).reshape(-1, 256)   # reshape copies already
    assert quant._row_stride(quant._as_2d(z)) == 256
    one = torch.randn(1, 2, 256)[:, 0]                 # one row, stride(0) = 512
    assert quant._row_stride(quant._as_2d(one)) == 256


def _rnd32(fr):
    """Round a rational to the nearest fp32 (ties to even, subnormals included), exactly."""
    from fractions import Fraction as F
    if fr == 0:
        return np.float32(0.0)
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while F(2) ** e > a:
        e -= 1
    while F(2) ** (e + 1) <= a:
        e += 1
    ulp = F(2) ** (max(e, -126) - 23)
    k, r = divmod(a / ulp, 1)
    k = int(k) + (1 if r > F(1, 2) or (r == F(1, 2) and int(k) % 2) else 0)
    return np.float32((1 if fr > 0 else -1) * float(k * ulp))


def test_fma_corrected_quotient_is_correctly_rounded():
    """The tensorwise kernels divide by the scale as q = fl(x y), y = fl(1 / scale), corrected by
    c = fl(q + fl(x - q scale) y) (two FMAs), then give c the sign of x, whenever amax lies in
    [2^-60, FLT_MAX]. In exact rational arithmetic, over random and adversarial x (scale times an
    fp8 grid value, one ulp off), amax at both ends of that range and x whose residual underflows:
    c is the correctly rounded quotient, or (|x| < 2^-102 only) both round to fp8 zero (quotient
    below 2^-26, under half the smallest e5m2 subnormal 2^-16)."""
    import random
    from fractions import Fraction as F
    rng = random.Random(5)
    fmaxes = [np.float32(448.0), np.float32(57344.0)]
    amaxes = [np.float32(2.0 ** -60), np.float32(3.4028235e38)]
    amaxes += [np.float32(abs(rng.gauss(0, 1)) * 2.0 ** rng.randint(-59, 120)) for _ in range(60)]
    n = 0
    for amax in amaxes:
        for fmax in fmaxes:
            s = _rnd32(F(float(amax)) / F(float(fmax)))
            y = _rnd32(F(1) / F(float(s)))
            xs = [amax, -amax, np.float32(2.0 ** -110), np.float32(-(2.0 ** -103) * 1.5), np.float32(1e-45)]
            for _ in range(20):
                xs.append(np.float32(rng.uniform(-1, 1) * float(amax)))
                g = _rnd32(F(float(s)) * rng.randint(1, 2 ** 10) / 2 ** rng.randint(0, 12))
                xs.append(np.nextafter(g, np.float32(np.inf if rng.random() < 0.5 else -np.inf), dtype=np.float32))
            for x in xs:
                if not (abs(x) <= amax):
                    continue
                q = np.float32(x * y)
                r = _rnd32(F(float(x)) - F(float(q)) * F(float(s)))
                c = _rnd32(F(float(r)) * F(float(y)) + F(float(q)))
                c = np.float32(np.copysign(c, x))
                exact = _rnd32(F(float(x)) / F(float(s)))
                if abs(x) < 2.0 ** -102:
                    assert abs(float(exact)) < 2.0 ** -26 and abs(float(c)) < 2.0 ** -26
                else:
                    assert c == exact and np.signbit(c) == np.signbit(x), (x, s, c, exact)
                n += 1
    assert n > 4000


def test_guarded_quotient_with_given_scale():
    """With a given scale (delayed scaling) the kernels compute q = fl(x y), y = fl(1 / scale); a q
    beyond 2 fmax goes to the clamp as it is, otherwise the FMA-corrected c (as above) does, for
    scales in [2^-80, 2^100]. In exact rational arithmetic, over scales at both ends and between,
    and x from far below the scale's range to far above it (overflowing products included),
    quotients near 2 fmax and fmax, and one-ulp-off grid values: the fp8 byte of clamp(result)
    equals that of clamp(correctly rounded x / scale)."""
    import random
    from fractions import Fraction as F
    from oracle import quant_oracle as orq
    rng = random.Random(9)
    scales = [np.float32(2.0 ** -80), np.float32(2.0 ** 100), np.float32(2.0 ** -80 * 1.9),
              np.float32(2.0 ** 99 * 1.7)]
    scales += [np.float32(abs(rng.gauss(0, 1)) * 2.0 ** rng.randint(-79, 99)) for _ in range(40)]
    n = 0
    for fmt in ("e4m3", "e5m2"):
        fmax = orq.FMAX[fmt]
        for s in scales:
            y = _rnd32(F(1) / F(float(s)))
            xs = [np.float32(2.0 ** -110), np.float32(-(2.0 ** -103) * 1.5), np.float32(1e-45),
                  np.float32(3.4e38), np.float32(-3.4e38)]
            for k in (2, 1):                                 # around 2 fmax (the guard) and fmax
                b = _rnd32(F(float(s)) * F(float(fmax)) * k)
                for d in range(-3, 4):
                    v = b
                    for _ in range(abs(d)):
                        v = np.nextafter(v, np.float32(np.inf if d > 0 else 0), dtype=np.float32)
                    xs += [v, -v]
            for _ in range(20):
                with np.errstate(over="ignore"):
                    xs.append(np.float32(rng.uniform(-1, 1) * float(s) * float(fmax) * 2.0 ** rng.randint(-30, 30)))
                g = _rnd32(F(float(s)) * rng.randint(1, 2 ** 10) / 2 ** rng.randint(0, 12))
                xs.append(np.nextafter(g, np.float32(np.inf if rng.random() < 0.5 else -np.inf), dtype=np.float32))
            for x in xs:
                if not np.isfinite(x):
                    continue
                with np.errstate(over="ignore"):
                    q = np.float32(x * y)
                if not (abs(q) <= 2 * fmax):
                    got = q
                else:
                    r = _rnd32(F(float(x)) - F(float(q)) * F(float(s)))
                    got = np.float32(np.copysign(_rnd32(F(float(r)) * F(float(y)) + F(float(q))), x))
                ex = F(float(x)) / F(float(s))
                exact = _rnd32(ex) if abs(ex) < F(2) ** 128 else np.float32(np.copysign(np.inf, x))
                b_got = orq.encode_fp8(orq._clamp(np.array([got], np.float32), fmt), fmt)[0]
                b_ref = orq.encode_fp8(orq._clamp(np.array([exact], np.float32), fmt), fmt)[0]
                if abs(x) < 2.0 ** -102:
                    assert b_got & 0x7F == 0 and b_ref & 0x7F == 0
                else:
                    assert b_got == b_ref, (fmt, x, s, got, exact)
                n += 1
    assert n > 4000
