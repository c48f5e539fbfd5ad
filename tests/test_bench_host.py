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


def _smi_doc(watts, clks, gpus=1):
    """An amd-smi metric -p -c --json document (the fields bench.py reads, with neighbours)."""
    import json
    gpu = {"gpu": 0, "power": {"socket_power": {"value": watts, "unit": "W"}, "gfx_voltage": "N/A"},
           "clock": {**{f"gfx_{i}": {"clk": {"value": c, "unit": "MHz"}, "max_clk": {"value": 2400, "unit": "MHz"}}
                        for i, c in enumerate(clks)},
                     "mem_0": {"clk": {"value": 1900, "unit": "MHz"}}, "fclk_0": {"clk": {"value": 2000, "unit": "MHz"}}}}
    return json.dumps({"gpu_data": [gpu] * gpus})


def test_parse_amd_smi():
    """Socket power and the mean of the XCDs' gfx clocks (memory and fabric clocks left out); a
    reading that lists several GPUs is refused, the list form is accepted."""
    import json
    w, mhz = bench.parse_amd_smi(_smi_doc(1394, [1860, 1880, 1870, 1870, 1860, 1880, 1870, 1870]))
    assert w == 1394.0 and mhz == 1870.0
    with pytest.raises(ValueError, match="2 GPUs"):
        bench.parse_amd_smi(_smi_doc(1394, [1870], gpus=2))
    doc = json.loads(_smi_doc(700, [2400, 2398]))["gpu_data"]
    assert bench.parse_amd_smi(json.dumps(doc)) == (700.0, 2399.0)


def test_summarize_power_middle_half():
    """Medians over the readings in the window's middle half only (the ramp of the first quarter and
    the tail are left out), error lines ignored; ms per launch from the window's wall time, energy
    per launch = power x ms; no reading inside -> an error record naming the last failure."""
    t0, t1 = 100.0, 108.0
    samples = [{"t": t0 + 0.25 * i, "watts": (900.0 if i < 8 else 1390.0 + (i % 3)), "mhz": 2000.0 if i < 8 else 1870.0}
               for i in range(32)]
    samples.insert(12, {"t": 104.0, "error": "TimeoutExpired"})
    rec = bench.summarize_power(samples, t0, t1, launches=5000)
    assert rec["watts"] == 1391.0 and rec["gfx_clock_mhz"] == 1870 and rec["cap_watts"] == 1400
    assert rec["ms_per_launch"] == 1.6 and rec["energy_per_launch_j"] == round(1391.0 * 1.6e-3, 3)
    assert rec["samples"] == 17 and rec["seconds"] == 8.0
    bad = bench.summarize_power([{"t": 104.0, "error": "FileNotFoundError: amd-smi"}], t0, t1, 10)
    assert bad == {"error": "FileNotFoundError: amd-smi"}


def test_power_sampler_child(tmp_path, monkeypatch):
    """The sampler protocol end to end on the CPU, with a stand-in amd-smi on PATH: the child
    records nothing before start(), readings once it is on, and stop() ends it and returns them."""
    import time
    fake = tmp_path / "amd-smi"
    fake.write_text("#!/bin/sh\ncat <<'EOF'\n" + _smi_doc(1234, [1900, 1910]) + "\nEOF\n")
    fake.chmod(0o755)
    monkeypatch.setenv("PATH", f"{tmp_path}:{__import__('os').environ['PATH']}")
    s = bench.PowerSampler(interval=0.05)
    try:
        time.sleep(0.5)
        import os
        assert os.path.getsize(s.path) == 0
        s.start()
        deadline = time.time() + 20
        while os.path.getsize(s.path) < 200 and time.time() < deadline:
            time.sleep(0.1)
    finally:
        samples = s.stop()
    assert s.proc.poll() is not None
    good = [x for x in samples if "watts" in x]
    assert len(good) >= 2 and all(x["watts"] == 1234.0 and x["mhz"] == 1905.0 for x in good), samples[:3]
