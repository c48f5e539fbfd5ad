"""The measured MFMA fixture (tests/golden/mfma_probe.npz) stays what the kernels compute: its inputs
re-run through the C ABI give the recorded outputs bit for bit (fp32 and bf16 wgrad with both
MFMA kernels, MX wgrad, persistent GEMM in both A formats). The CPU test tests/test_oracle_mfma.py
pins the error model against the same recorded outputs."""
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
