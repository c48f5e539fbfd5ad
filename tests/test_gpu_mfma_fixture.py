"""The measured MFMA fixture (tests/golden/mfma_probe.npz) stays what the kernels compute: its inputs
re-run through the C ABI give the recorded outputs bit for bit (fp32 and bf16 wgrad with both
MFMA kernels, MX wgrad, persistent GEMM in both A formats; and the sampled outputs of the wide-tile
kernels). The CPU test tests/test_oracle_mfma.py pins the error model against the same recorded
outputs."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def test_fixture_outputs_reproduce(pkg, cuda):
    path = os.path.join(GOLDEN, "mfma_probe.npz")
    if not os.path.exists(path):
        pytest.skip("fixture not written yet")
    print("[gpu-case] mfma fixture re-run", flush=True)
    z = np.load(path)
    one = torch.tensor(1.0, dtype=torch.float32, device=cuda)
    t = lambda k: torch.from_numpy(z[k]).to(cuda)
    f32 = pkg.grouped_gemm_fp8_tensorwise_variable_k(t("wg_lhs"), t("wg_rhs"), one, one, t("wg_offs"),
                                                     out_dtype=torch.float32)
    b128 = pkg.grouped_gemm_fp8_tensorwise_variable_k(t("wg_lhs"), t("wg_rhs"), one, one, t("wg_offs"))
    b32 = pkg.grouped_gemm_fp8_tensorwise_variable_k(t("wg_lhs"), t("wg_rhs"), one, one, t("wg_offs"), mfma="k32")
    mx = pkg.grouped_gemm_mxfp8_variable_k(t("mx_lhs"), t("mx_rhs"), t("mx_lsc"), t("mx_rsc"), t("mx_offs"))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(f32.cpu().numpy().view(np.uint32), z["wg_out_f32"].view(np.uint32))
    np.testing.assert_array_equal(pkg.as_bf16_bits(b128), z["wg_out_bf16_k128"])
    np.testing.assert_array_equal(pkg.as_bf16_bits(b32), z["wg_out_bf16_k32"])
    np.testing.assert_array_equal(pkg.as_bf16_bits(mx), z["mx_out_bf16"])
    for fmt in ("e4m3", "e5m2"):
        adt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
        out = pkg.grouped_gemm_fp8_tensorwise(t(f"p_a_{fmt}").view(adt), t("p_b").view(torch.float8_e4m3fn), one, one,
                                              t("p_offs"))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(pkg.as_bf16_bits(out), z[f"p_out_bf16_{fmt}"])


def _sample(a, rows, cols):
    return a[:, rows][:, :, cols]


def test_fixture_wide_outputs_reproduce(pkg, cuda):
    """The wide-tile kernels' recorded samples (320 x 320 bf16 / fp32 / fp32 accumulate, 256 x 384,
    the MX 320 x 320 kernel, the wide persistent kernel in both A formats) re-run bit for bit."""
    path = os.path.join(GOLDEN, "mfma_probe.npz")
    z = np.load(path)
    if "w320_out_bf16" not in z:
        pytest.skip("fixture has no wide-kernel entries yet")
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_mfma_fixture", os.path.join(GOLDEN, "make_mfma_fixture.py"))
    fx = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(fx)
    print("[gpu-case] mfma fixture re-run, wide kernels", flush=True)
    one = torch.tensor(1.0, dtype=torch.float32, device=cuda)
    t = lambda k: torch.from_numpy(z[k]).to(cuda)
    run = pkg.grouped_gemm_fp8_tensorwise_variable_k
    R, C = fx.W320_ROWS, fx.W320_COLS
    b = run(t("w320_lhs"), t("w320_rhs"), one, one, t("w320_offs"), wide=320)
    f = run(t("w320_lhs"), t("w320_rhs"), one, one, t("w320_offs"), out_dtype=torch.float32, wide=320)
    c0 = np.zeros((z["w320_offs"].size - 1, 320, 320), np.float32)
    c0[:, R[:, None], C[None, :]] = z["w320_c0"]
    acc = torch.from_numpy(c0).to(cuda)
    run(t("w320_lhs"), t("w320_rhs"), one, one, t("w320_offs"), out=acc, accumulate=True, wide=320)
    b256 = run(t("w256_lhs"), t("w256_rhs"), one, one, t("w256_offs"), wide=256)
    mx = pkg.grouped_gemm_mxfp8_variable_k(t("w320mx_lhs"), t("w320mx_rhs"), t("w320mx_lsc"), t("w320mx_rsc"),
                                           t("w320mx_offs"), tile_m=320)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_sample(pkg.as_bf16_bits(b), R, C), z["w320_out_bf16"])
    np.testing.assert_array_equal(_sample(f.cpu().numpy(), R, C).view(np.uint32), z["w320_out_f32"].view(np.uint32))
    np.testing.assert_array_equal(_sample(acc.cpu().numpy(), R, C).view(np.uint32),
                                  z["w320_out_f32_acc"].view(np.uint32))
    np.testing.assert_array_equal(_sample(pkg.as_bf16_bits(b256), fx.W256_ROWS, fx.W384_COLS), z["w256_out_bf16"])
    np.testing.assert_array_equal(_sample(pkg.as_bf16_bits(mx), R, C), z["w320mx_out_bf16"])
    for fmt in ("e4m3", "e5m2"):
        adt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
        out = pkg.grouped_gemm_fp8_tensorwise(t(f"wp_a_{fmt}").view(adt), t("wp_b").view(torch.float8_e4m3fn), one,
                                              one, t("wp_offs"), kernel="wide")
        torch.cuda.synchronize()
        np.testing.assert_array_equal(pkg.as_bf16_bits(out)[:, C], z[f"wp_out_bf16_{fmt}"])
