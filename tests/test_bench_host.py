"""CPU tests of bench.py's checker: the oracle leg that compares the last timed launch's output
with the oracle over every group (the reference checks the kernel it times in the same harness,
reference bench.py:594-648, cosine at :641-646). The checker must accept an exact result, accept a
result within the bar, and reject each kind of mistake the bar names: one element off by more than
2e-2 relative, a non-finite value, a non-zero empty group, a wrong group (the cosine)."""
import sys

import numpy as np
import pytest
import torch

import bench


@pytest.fixture(scope="module")
def plumbing(pkg):
    return pkg.inputs.make_problem("plumbing", seed=0, device="cpu")


@pytest.fixture(scope="module")
def exact(plumbing, orc):
    p = plumbing
    bits = orc.vark_wgrad_tensorwise(p.lhs.numpy(), p.rhs.numpy(), p.lhs_scale, p.rhs_scale, p.group_offs.numpy())
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)


def _leg(p, out, seconds=0.0):
    par, base = bench.oracle_leg(p, {"library": out}, seconds)
    return par["library"], base


def test_exact_output_passes(plumbing, exact):
    m, base = _leg(plumbing, exact.clone(), seconds=5.0)
    assert m["ok"] and m["exact_frac"] == 1.0 and m["groups"] == "4 of 4"
    assert m["empty_groups"] == 1 and m["empty_zero"]
    # the timed sample covers the non-empty groups (3 of 4) within the budget
    assert base is not None and base["unit"] == "TFLOPS" and base["sample"].startswith("3 of 4 groups")


def test_fp32_output_rounded_to_bf16_passes(plumbing, exact):
    m, _ = _leg(plumbing, exact.float())
    assert m["ok"] and m["exact_frac"] == 1.0


def test_output_within_the_bar_passes(plumbing, exact):
    out = exact.float() * (1 + 2.0 ** -7)     # one to two bf16 ulps
    m, _ = _leg(plumbing, out.to(torch.bfloat16))
    assert m["ok"] and 0 < m["max_rel"] <= 2e-2


def test_one_element_off_fails(plumbing, exact):
    out = exact.clone()
    g, i, j = 3, 5, 7
    out[g, i, j] = out[g, i, j] * 1.05 if abs(float(out[g, i, j])) > 0 else out[g].float().abs().max()
    m, _ = _leg(plumbing, out)
    assert not m["ok"] and m["max_rel"] > 2e-2 and m["cos"] > 0.99999   # the cosine alone would pass it


def test_nonfinite_fails(plumbing, exact):
    out = exact.clone()
    out[1, 0, 0] = float("nan")
    m, _ = _leg(plumbing, out)
    assert not m["ok"] and m["nonfinite"] == 1


def test_nonzero_empty_group_fails(plumbing, exact):
    out = exact.clone()
    out[2, 3, 4] = 1e-30     # group 2 is empty: any non-zero bit pattern fails
    m, _ = _leg(plumbing, out)
    assert not m["ok"] and not m["empty_zero"]


def test_swapped_groups_fail(plumbing, exact):
    out = exact.clone()
    out[[0, 1]] = out[[1, 0]]
    m, _ = _leg(plumbing, out)
    assert not m["ok"] and m["cos"] < 0.99999


def test_no_baseline_without_cpu_seconds(plumbing, exact):
    _, base = _leg(plumbing, exact.clone(), seconds=0.0)
    assert base is None


def test_fwd_leg(pkg, orp, orc):
    p = pkg.inputs.make_fwd_problem("down_fwd", seed=0, device="cpu", lens=torch.tensor([40, 0, 88]), K=64, N=48)
    ref = orp.grouped_fp8(p.a.numpy(), p.b.numpy(), p.a_scale, p.b_scale, p.group_offs.numpy(), p.a_format)
    out = torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16)
    bad = out.clone()
    bad[100, 3] = -bad[100, 3] if float(bad[100, 3]) != 0 else 1.0
    par, base = bench.oracle_leg_fwd(p, {"library": out.clone(), "drop_in_co": bad}, 5.0)
    m = par["library"]
    assert m["ok"] and m["exact_frac"] == 1.0 and m["groups"] == "3 of 3 (128 rows)" and base is not None
    assert not par["drop_in_co"]["ok"]


def test_power_record_for_measured_variants_only(monkeypatch):
    """The roofline object's power record: the default line (gate_up_wgrad, bf16 C, multinomial
    lengths) and the other measured variants map to their rows of profiles/power_sites.txt, whose
    figures parse; unmeasured variants get none."""
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    args = bench.parse_args()
    assert bench.power_label(args) == "gate_up_wgrad, bf16 C"
    rec = bench.read_power(bench.power_label(args))
    assert rec is not None and rec["cap_watts"] == 1400
    assert 1000 < rec["watts"] <= 1400 and 1000 < rec["gfx_clock_mhz"] <= 2400 and rec["energy_per_launch_j"] > 0
    for argv, want in ((["--out", "f32_accum", "--lens", "reference"], "gate_up_wgrad, fp32 accumulate (ref)"),
                       (["--config", "gate_up_fwd"], "gate_up_fwd, contiguous rows"),
                       (["--config", "gate_up_fwd", "--row-align", "128"], "gate_up_fwd, 128-byte rows"),
                       (["--config", "gate_up_fwd", "--persistent-kernel", "512"], "gate_up_fwd, 512-thread kernel"),
                       (["--out", "f32_accum"], None), (["--mfma", "k32"], None), (["--config", "down_fwd"], None)):
        monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
        a = bench.parse_args()
        assert bench.power_label(a) == want, argv
        if want:
            assert bench.read_power(want) is not None, want
    assert bench.read_power("no such row") is None
