"""Writes tests/golden/plumbing_g4_m512.npz: BASELINE config 1 (G=4, M_total=512, group sizes
[96, 160, 0, 256], LHS e4m3 [512, 64] with scale amax/448, RHS e5m2 [512, 128] with scale
amax/57344, seed 0) and the CPU oracle's bf16 output. Run from the repo root:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from __graft_entry__ import load_package  # noqa: E402
from oracle import vark_oracle as orc  # noqa: E402


def main():
    pkg = load_package()
    prob = pkg.inputs.make_problem("plumbing", seed=0, device="cpu")
    lhs, rhs, offs = prob.lhs.numpy(), prob.rhs.numpy(), prob.group_offs.numpy()
    sl, sr = np.float32(prob.lhs_scale), np.float32(prob.rhs_scale)
    bits = orc.vark_wgrad_tensorwise(lhs, rhs, sl, sr, offs)
    out = os.path.join(ROOT, "tests", "golden", "plumbing_g4_m512.npz")
    np.savez_compressed(out, lhs=lhs, rhs=rhs, group_offs=offs, lhs_scale=sl, rhs_scale=sr,
                        expected_bf16_bits=bits)
    print(f"wrote {out}: {os.path.getsize(out)} bytes")


if __name__ == "__main__":
    main()
