"""Writes mfma_probe.npz: inputs and the GPU's measured outputs that pin the fp8 MFMA accumulation
model (oracle.vark_oracle.fp8_mfma_emulate / fp8_mfma_error_bound) on the CPU.

Runs on an MI355X (the outputs are measured, not computed): from the repo root,
    python tests/golden/make_mfma_fixture.py [OUT.npz]
(default tests/golden/mfma_probe.npz). Every launch goes through the library's C ABI; the CPU test
tests/test_oracle_mfma.py reads the file, and tests/test_gpu_mfma_fixture.py re-runs the same
inputs and requires the same bits.

Cases (finite fp8 codes only; scales 1.0, so the fp32-output mode returns the raw accumulator):
  * wgrad, G = 5, OUT_M = 32, OUT_N = 48, group sizes [128, 37, 0, 300, 160]:
    - group 0: column (0, 0) is the known answer 2^6 + 127 * 2^-8 (token 0 holds 8.0 on both
      sides, every other token 2^-4); the other columns hold random codes;
    - groups 1, 3: uniformly random finite codes (every exponent, both signs);
    - group 4: the configured value recipe (N(0,1) and N(0,1e-3) quantized per tensor);
    outputs: fp32 (K=128 MFMA kernel), bf16 (K=128) and bf16 (K=32 MFMA kernel).
  * MX wgrad, group sizes [64, 96], OUT 32 x 48, random codes and random e8m0 scales 120..134:
    bf16 output.
  * persistent fwd/dgrad GEMM, both A formats, rows [100, 200], K = 128 + 64 (a K tail), N = 48,
    random codes: bf16 output.
The same cases on the wide-tile kernels (the unscaled and scaled v_mfma_f32_32x32x64_f8f6f4), each
recording a sample of output rows and columns that covers every wave's quadrant of a tile (an
element depends only on its own operand row and column, so the inputs are zero outside the sampled
columns and the file stays small):
  * wgrad on the 320 x 320 kernel (OUT 320 x 320; rows/columns 0-31 and 160-191, columns 288-319
    too; the wgrad group sizes and value kinds above, the known answer at (0, 0, 0)): bf16, fp32,
    and fp32 accumulate into a recorded C0;
  * wgrad on the 256 x 384 kernel (OUT 256 x 384; rows 0-31 and 128-159, columns 0-31, 192-223 and
    352-383): bf16;
  * MX wgrad on the 320 x 320 MX kernel (OUT 320 x 320, group sizes [64, 96], random codes and
    e8m0 scales 120..134): bf16;
  * persistent GEMM on the wide kernel (256 x 320 tiles; rows [100, 200], K = 256, N = 320, both A
    formats, random codes; all rows, columns 0-31, 160-191, 288-319): bf16.
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from __graft_entry__ import load_package  # noqa: E402


def _codes(rng, shape, fmt):
    c = rng.integers(0, 256, shape, dtype=np.uint8)
    if fmt == "e4m3":
        c[(c & 0x7F) == 0x7F] = 0x3A       # NaN codes -> 1.25
    else:
        c[(c & 0x7C) == 0x7C] = 0x3B       # inf / NaN codes -> 0.875
    return c


def _recipe(rng, rows, cols, fmt):
    x = torch.from_numpy(rng.standard_normal((rows, cols)).astype(np.float32))
    if fmt == "e5m2":
        x = x * 1e-3
    fmax = 448.0 if fmt == "e4m3" else 57344.0
    scale = float(x.abs().max()) / fmax
    dt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    return (x / scale).clamp(-fmax, fmax).to(dt).view(torch.uint8).numpy()


# sampled output rows / columns of the wide kernels: both waves of a tile in each dimension, and the
# last block column of the 320-wide tile
W320_ROWS = np.r_[0:32, 160:192]
W320_COLS = np.r_[0:32, 160:192, 288:320]
W256_ROWS = np.r_[0:32, 128:160]
W384_COLS = np.r_[0:32, 192:224, 352:384]


def _only(cols, arr):
    """arr with every column outside ``cols`` zeroed (last axis)."""
    out = np.zeros_like(arr)
    out[..., cols] = arr[..., cols]
    return out


def _wgrad_inputs(rng, lens, om, on, rows, cols):
    """The wgrad fixture's inputs (known answer in group 0 at (0, 0), random codes in groups 1 and
    3, the value recipe in group 4), zero outside the sampled columns."""
    M = sum(lens)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    lhs = _codes(rng, (M, om), "e4m3")
    rhs = _codes(rng, (M, on), "e5m2")
    lhs[0:128, 0] = 0x18
    rhs[0:128, 0] = 0x2C
    lhs[0, 0] = 0x50
    rhs[0, 0] = 0x48
    o4, o5 = offs[4], offs[5]
    lhs[o4:o5] = _recipe(rng, o5 - o4, om, "e4m3")
    rhs[o4:o5] = _recipe(rng, o5 - o4, on, "e5m2")
    return _only(rows, lhs), _only(cols, rhs), offs


def wide_cases(pkg, dev, z):
    rng = np.random.default_rng(20261203)
    one = torch.tensor(1.0, dtype=torch.float32, device=dev)
    lens = [128, 37, 0, 300, 160]
    T = lambda a: torch.from_numpy(a).to(dev)
    run = pkg.grouped_gemm_fp8_tensorwise_variable_k
    sample = lambda t, r, c: t.cpu()[:, r][:, :, c].numpy()

    # ---- 320 x 320 kernel: bf16, fp32, fp32 accumulate
    lhs, rhs, offs = _wgrad_inputs(rng, lens, 320, 320, W320_ROWS, W320_COLS)
    dl, dr, do = T(lhs), T(rhs), T(offs)
    b = run(dl, dr, one, one, do, wide=320)
    f = run(dl, dr, one, one, do, out_dtype=torch.float32, wide=320)
    c0 = np.zeros((len(lens), 320, 320), np.float32)
    c0[:, W320_ROWS[:, None], W320_COLS[None, :]] = rng.standard_normal((len(lens), 64, 96)).astype(np.float32)
    acc = T(c0)
    run(dl, dr, one, one, do, out=acc, accumulate=True, wide=320)
    torch.cuda.synchronize()
    z.update(w320_lhs=lhs, w320_rhs=rhs, w320_offs=offs, w320_c0=c0[:, W320_ROWS][:, :, W320_COLS],
             w320_out_bf16=pkg.as_bf16_bits(b)[:, W320_ROWS][:, :, W320_COLS],
             w320_out_f32=sample(f, W320_ROWS, W320_COLS), w320_out_f32_acc=sample(acc, W320_ROWS, W320_COLS))
    print(f"wide320 known answer (0, 0, 0): {float(f[0, 0, 0])!r}", flush=True)

    # ---- 256 x 384 kernel: bf16
    lhs, rhs, offs = _wgrad_inputs(rng, lens, 256, 384, W256_ROWS, W384_COLS)
    b = run(T(lhs), T(rhs), one, one, T(offs), wide=256)
    torch.cuda.synchronize()
    z.update(w256_lhs=lhs, w256_rhs=rhs, w256_offs=offs,
             w256_out_bf16=pkg.as_bf16_bits(b)[:, W256_ROWS][:, :, W384_COLS])

    # ---- MX on the 320 x 320 kernel
    mlens = [64, 96]
    mM = sum(mlens)
    moffs = np.concatenate([[0], np.cumsum(mlens)]).astype(np.int64)
    mlhs = _only(W320_ROWS, _codes(rng, (mM, 320), "e4m3"))
    mrhs = _only(W320_COLS, _codes(rng, (mM, 320), "e5m2"))
    lsc = rng.integers(120, 135, (mM // 32, 320), dtype=np.uint8)
    rsc = rng.integers(120, 135, (mM // 32, 320), dtype=np.uint8)
    mx = pkg.grouped_gemm_mxfp8_variable_k(T(mlhs), T(mrhs), T(lsc), T(rsc), T(moffs), tile_m=320)
    torch.cuda.synchronize()
    z.update(w320mx_lhs=mlhs, w320mx_rhs=mrhs, w320mx_lsc=lsc, w320mx_rsc=rsc, w320mx_offs=moffs,
             w320mx_out_bf16=pkg.as_bf16_bits(mx)[:, W320_ROWS][:, :, W320_COLS])

    # ---- persistent GEMM on the wide kernel, both A formats
    plens = [100, 200]
    pM, K, N = sum(plens), 256, 320
    poffs = np.concatenate([[0], np.cumsum(plens)]).astype(np.int64)
    pb = _codes(rng, (len(plens), N, K), "e4m3")
    keep = np.zeros(N, bool)
    keep[W320_COLS] = True
    pb[:, ~keep, :] = 0
    z.update(wp_offs=poffs, wp_b=pb)
    for fmt in ("e4m3", "e5m2"):
        a = _codes(rng, (pM, K), fmt)
        adt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
        out = pkg.grouped_gemm_fp8_tensorwise(T(a).view(adt), T(pb).view(torch.float8_e4m3fn), one, one, T(poffs),
                                              kernel="wide")
        torch.cuda.synchronize()
        z[f"wp_a_{fmt}"] = a
        z[f"wp_out_bf16_{fmt}"] = pkg.as_bf16_bits(out)[:, W320_COLS]


def main(path):
    pkg = load_package()
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(20261202)
    one = torch.tensor(1.0, dtype=torch.float32, device=dev)
    z = {}

    # ---- tensorwise wgrad
    lens = [128, 37, 0, 300, 160]
    om, on = 32, 48
    M = sum(lens)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    lhs = _codes(rng, (M, om), "e4m3")
    rhs = _codes(rng, (M, on), "e5m2")
    lhs[0:128, 0] = 0x18                   # 2^-4 (e4m3)
    rhs[0:128, 0] = 0x2C                   # 2^-4 (e5m2)
    lhs[0, 0] = 0x50                       # 8.0
    rhs[0, 0] = 0x48                       # 8.0
    o4, o5 = offs[4], offs[5]
    lhs[o4:o5] = _recipe(rng, o5 - o4, om, "e4m3")
    rhs[o4:o5] = _recipe(rng, o5 - o4, on, "e5m2")
    dl, dr, do = (torch.from_numpy(lhs).to(dev), torch.from_numpy(rhs).to(dev), torch.from_numpy(offs).to(dev))
    f32 = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, one, one, do, out_dtype=torch.float32)
    b128 = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, one, one, do)
    b32 = pkg.grouped_gemm_fp8_tensorwise_variable_k(dl, dr, one, one, do, mfma="k32")
    torch.cuda.synchronize()
    z.update(wg_lhs=lhs, wg_rhs=rhs, wg_offs=offs, wg_out_f32=f32.cpu().numpy(),
             wg_out_bf16_k128=pkg.as_bf16_bits(b128), wg_out_bf16_k32=pkg.as_bf16_bits(b32))
    print(f"wgrad known answer (0, 0, 0): {float(f32[0, 0, 0])!r} (exact {64 + 127 * 2.0 ** -8!r})", flush=True)

    # ---- MX wgrad
    mlens = [64, 96]
    mM = sum(mlens)
    moffs = np.concatenate([[0], np.cumsum(mlens)]).astype(np.int64)
    mlhs = _codes(rng, (mM, om), "e4m3")
    mrhs = _codes(rng, (mM, on), "e5m2")
    lsc = rng.integers(120, 135, (mM // 32, om), dtype=np.uint8)
    rsc = rng.integers(120, 135, (mM // 32, on), dtype=np.uint8)
    mx = pkg.grouped_gemm_mxfp8_variable_k(torch.from_numpy(mlhs).to(dev), torch.from_numpy(mrhs).to(dev),
                                           torch.from_numpy(lsc).to(dev), torch.from_numpy(rsc).to(dev),
                                           torch.from_numpy(moffs).to(dev))
    torch.cuda.synchronize()
    z.update(mx_lhs=mlhs, mx_rhs=mrhs, mx_lsc=lsc, mx_rsc=rsc, mx_offs=moffs, mx_out_bf16=pkg.as_bf16_bits(mx))

    # ---- persistent GEMM, both A formats
    plens = [100, 200]
    pM, K, N = sum(plens), 192, 48
    poffs = np.concatenate([[0], np.cumsum(plens)]).astype(np.int64)
    b = _codes(rng, (len(plens), N, K), "e4m3")
    z.update(p_offs=poffs, p_b=b)
    for fmt in ("e4m3", "e5m2"):
        a = _codes(rng, (pM, K), fmt)
        adt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
        out = pkg.grouped_gemm_fp8_tensorwise(torch.from_numpy(a).to(dev).view(adt),
                                              torch.from_numpy(b).to(dev).view(torch.float8_e4m3fn), one, one,
                                              torch.from_numpy(poffs).to(dev))
        torch.cuda.synchronize()
        z[f"p_a_{fmt}"] = a
        z[f"p_out_bf16_{fmt}"] = pkg.as_bf16_bits(out)

    wide_cases(pkg, dev, z)
    np.savez_compressed(path, **z)
    print(f"wrote {path}: {os.path.getsize(path)} bytes", flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else os.path.join(ROOT, "tests", "golden", "mfma_probe.npz"))
