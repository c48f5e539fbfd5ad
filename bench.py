#!/usr/bin/env python3
"""Benchmark of the FP8 grouped GEMMs on one MI355X.

Workload (BASELINE headline, the default): gate_up_wgrad, G=32 experts, M_total=131072 tokens,
LHS e4m3 [131072, 2880], RHS e5m2 [131072, 5760], C bf16 [32, 2880, 5760], per-tensor scales,
seeded uniform-multinomial group sizes, inputs generated directly in HBM. One step = one launch of
the grouped wgrad (all 32 experts). FLOPs per step = 2 * M_total * OUT_M * OUT_N (reference
bench.py:742, launcher.cpp:76).

``--config gate_up_fwd | down_fwd | down_dgrad | gate_up_dgrad`` measures the persistent
forward / data-gradient grouped GEMM at the reference's other call sites instead (reference
bench.py:153-180, inputs as in bench.py:205-223,238-247; FLOPs = 2 * M_total * K * N).

``--config gate_up_layer`` measures one training step of the FP8 grouped linear layer at the
gate_up shape (x bf16 [131072, 2880], w bf16 [32, 5760, 2880], dy bf16 [131072, 5760]): quantize
x and w, forward GEMM, quantize dy, dgrad GEMM, wgrad GEMM accumulated into an fp32 main-grad;
FLOPs = 3 * 2 * M * K * N. ``--scaling delayed`` quantizes x, w and dy with delayed scaling (scale
from an amax history, amax recorded in the quantizing pass: no amax pass in the step).

``--site all | all_fwd | all_wgrad | <site>`` runs the reference's call sites one after the other
with its own input recipe and prints its summary table (per-site ms, TFLOPS, share of the total)
on stderr; the JSON line carries the sum over the sites (reference bench.py:690-858).

``--config gate_up_ep8 | gate_up_ncol8 | gate_up_ncol6`` measures one GPU's share of gate_up_wgrad
when the path is sharded without communication: 8-way expert sharding (G = 4, M_total = 65536,
~16 K tokens per expert, 2880 x 5760) and N-column sharding (G = 32, M_total = 131072, OUT_N = 720
for 8 GPUs, 960 for 6).

``--config quant_tensorwise | quant_mx`` measures the FP8 quantization producer (HBM-bound, GB/s):
x bf16 [131072, 2880] -> per-tensor e4m3 (amax pass + quantize pass: 2 + 2 + 1 bytes per
element), and dy bf16 [131072, 5760] -> grouped MX e5m2 with 32-token padding (2 + 1 + 1/32
bytes per element). ``--config quant_weight_transpose``: w bf16 [32, 5760, 2880] -> e4m3 q and its
per-expert transpose q^T in one pass (2 + 2 + 1 + 1 bytes per element). The ``_delayed`` variants
of quant_tensorwise and quant_weight_transpose quantize with delayed scaling (scale from an amax
history of 16, the amax reduced in the quantizing pass: 2 + 1 and 2 + 1 + 1 bytes per element).

Prints ONE JSON line with ms, TFLOPS, the MFMA roofline fraction and a CPU baseline (the
build's numpy oracle on a bounded sample of the same workload, timed on this host's cores).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP8_DENSE_PEAK_TFLOPS = 5000.0    # MI355X dense FP8 MFMA peak
REF_OPT_ASM_TFLOPS = 1237.0       # reference optimized ASM, gate_up_wgrad, C launcher (README.md:60)
FWD_SITES = ("gate_up_fwd", "down_fwd", "down_dgrad", "gate_up_dgrad")
QUANT_CONFIGS = ("quant_tensorwise", "quant_mx", "quant_weight_transpose", "quant_tensorwise_delayed",
                 "quant_weight_transpose_delayed")
LAYER_CONFIGS = ("gate_up_layer",)
# one GPU's share of the gate_up wgrad when the path is sharded without communication: expert
# sharding over 8 GPUs (4 of the 32 experts, ~16 K routed tokens each) and N-column sharding (a
# slice of RHS and C, LHS replicated) over 8 GPUs (720 columns) or 6 (960 columns: three 320-wide tiles)
SHARD_CONFIGS = {"gate_up_ep8": dict(G=4, M=65536), "gate_up_ncol8": dict(OUT_N=720),
                 "gate_up_ncol6": dict(OUT_N=960)}
WGRAD_SITES = ("down_wgrad", "gate_up_wgrad")
SITE_GROUPS = {"all": (*FWD_SITES, *WGRAD_SITES), "all_fwd": FWD_SITES, "all_wgrad": WGRAD_SITES}
HBM_PEAK_GBS = 8000.0             # MI355X HBM3E


def traffic_file(name):
    return os.path.join(ROOT, "profiles", f"traffic_{name}.txt")


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="gate_up_wgrad",
                    choices=["gate_up_wgrad", "down_wgrad", "gate_up_zipf", "gate_up_mx", "plumbing", "constant",
                             *FWD_SITES, *QUANT_CONFIGS, *LAYER_CONFIGS, *SHARD_CONFIGS])
    ap.add_argument("--site", default=None, choices=[*SITE_GROUPS, *FWD_SITES, *WGRAD_SITES],
                    help="time the reference's call sites (one, or a group) with its own input recipe and print "
                         "a per-site summary table; replaces --config")
    ap.add_argument("--mfma", default="k128", choices=["k128", "k32"])
    ap.add_argument("--persistent-kernel", default="auto", choices=["auto", "512", "wide"],
                    help="fwd / dgrad sites: the library's kernel choice, or the 512-thread or the wide-tile "
                         "persistent kernel forced")
    ap.add_argument("--row-align", type=int, default=0,
                    help="fwd / dgrad sites: copy A and B into buffers whose row strides are multiples of this "
                         "many bytes (128: row segments on whole lines, the autograd op's layout); 0 keeps the "
                         "reference's contiguous inputs")
    ap.add_argument("--out", default="bf16", choices=["bf16", "f32", "f32_accum"],
                    help="tensorwise wgrad configs: C bf16, fp32, or fp32 accumulated in place (C += result)")
    ap.add_argument("--lens", default="multinomial", choices=["multinomial", "reference"],
                    help="tensorwise wgrad configs: the configuration's group sizes, or the reference's seed-42 "
                         "exponential ones (reference bench.py:205-223)")
    ap.add_argument("--scaling", default="current", choices=["current", "delayed"],
                    help="gate_up_layer: x, w and dy quantized with their own amax (an amax pass each), or with "
                         "delayed scaling (an amax history of 16; the amax reduced in the quantizing pass)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU work for the cpu_baseline sample (0 disables)")
    ap.add_argument("--no-parity", dest="parity", action="store_false",
                    help="skip the check of the last timed launch's output against the oracle over every group "
                         "(on by default; a failed bar exits with status 1)")
    ap.add_argument("--no-drop-in", dest="drop_in", action="store_false",
                    help="tensorwise wgrad configs: do not time the drop-in code object beside the library")
    ap.add_argument("--drop-in-steps", type=int, default=None,
                    help="timed launches of the drop-in code object (default: --steps)")
    ap.add_argument("--power-seconds", type=float, default=0.0,
                    help="after timing, launch the step back to back for this long while amd-smi samples the "
                         "board's power and gfx clock (every 0.25 s, from a child process started before the GPU "
                         "is touched); the medians of the window's middle half go into roofline.power (or "
                         "drop_in_co.power with --power-of drop_in) in place of the recorded figures")
    ap.add_argument("--power-of", default="library", choices=["library", "drop_in"],
                    help="what the power window launches: the library step or the drop-in code object")
    ap.add_argument("--power-sampler", default=None, help=argparse.SUPPRESS)   # child-process mode
    ap.add_argument("--power-interval", type=float, default=POWER_INTERVAL_S, help=argparse.SUPPRESS)
    ap.add_argument("--extra", action="store_true", help="also time the other configs (not part of the line)")
    ap.add_argument("--info", action="store_true",
                    help="print the registers, spills, LDS and MFMA counts of this build's code objects and exit "
                         "(no GPU needed)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only run a plain device-to-device copy of this many MiB (steps times): the "
                         "known-size reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


def copy_calibration(mib, steps):
    import torch
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": mib << 20, "launches": steps}), flush=True)


def read_traffic(name):
    """(HBM bytes per launch, where they come from): the rocprofv3 --pmc measurement (FETCH_SIZE +
    WRITE_SIZE, calibrated) recorded in profiles/traffic_<name>.txt with the kernel revision it was
    taken at, or (None, None). Not measured by this run."""
    value, rev = None, None
    try:
        for line in open(traffic_file(name)):
            if line.startswith("traffic_bytes_per_launch:"):
                value = float(line.split(":", 1)[1])
            elif line.startswith("kernel_revision:"):
                rev = line.split(":", 1)[1].strip()
    except OSError:
        return None, None
    src = f"profiles/traffic_{name}.txt (rocprofv3 --pmc, kernel revision {rev or 'unrecorded'})"
    return value, (src if value is not None else None)


POWER_FILE = os.path.join(ROOT, "profiles", "power_sites.txt")
POWER_CAP_W = 1400                # MI355X rated board power; amd-smi metric reports no limit
POWER_INTERVAL_S = 0.25


def parse_amd_smi(text):
    """(socket power in W, mean gfx clock over the XCDs in MHz) from one ``amd-smi metric -p -c
    --json`` document of a single GPU."""
    d = json.loads(text)
    gpus = d["gpu_data"] if isinstance(d, dict) else d
    if len(gpus) != 1:
        raise ValueError(f"amd-smi lists {len(gpus)} GPUs; this reading needs exactly the one in use")
    g = gpus[0]
    clks = [float(v["clk"]["value"]) for k, v in g["clock"].items()
            if k.startswith("gfx_") and isinstance(v, dict) and isinstance(v.get("clk"), dict)]
    if not clks:
        raise ValueError("no gfx clock in the amd-smi reading")
    return float(g["power"]["socket_power"]["value"]), sum(clks) / len(clks)


def power_sampler(path, interval):
    """Body of ``bench.py --power-sampler PATH``: a child process that the parent starts before it
    touches the GPU and that never touches it itself. Once PATH + ".go" exists it appends one line
    per ``amd-smi metric -p -c --json`` reading to PATH, ``{"t": unix time, "watts", "mhz"}`` or
    ``{"t", "error"}``, every ``interval`` s, until the parent terminates it or exits."""
    import subprocess
    parent = os.getppid()
    while os.getppid() == parent and not os.path.exists(path + ".go"):
        time.sleep(0.05)
    with open(path, "a") as f:
        while os.getppid() == parent:
            t = time.time()
            try:
                r = subprocess.run(["amd-smi", "metric", "-p", "-c", "--json"], capture_output=True, text=True,
                                   timeout=10)
                watts, mhz = parse_amd_smi(r.stdout)
                rec = {"t": round(t, 3), "watts": watts, "mhz": round(mhz, 1)}
            except Exception as e:   # a missing tool or an unexpected document: recorded, not fatal
                rec = {"t": round(t, 3), "error": f"{type(e).__name__}: {e}"[:200]}
            f.write(json.dumps(rec) + "\n")
            f.flush()
            time.sleep(interval)


class PowerSampler:
    """Parent side of ``power_sampler``: started before the GPU is touched (a process that has
    initialised the GPU starts no other program), switched on for the power window only."""

    def __init__(self, interval=POWER_INTERVAL_S):
        import subprocess
        import tempfile
        fd, self.path = tempfile.mkstemp(prefix="ggemm_power_", suffix=".jsonl")
        os.close(fd)
        self.proc = subprocess.Popen([sys.executable, os.path.abspath(__file__), "--power-sampler", self.path,
                                      "--power-interval", str(interval)],
                                     stdin=subprocess.DEVNULL, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)

    def start(self):
        open(self.path + ".go", "w").close()

    def stop(self):
        """End the child; its readings as dicts."""
        self.proc.terminate()
        try:
            self.proc.wait(timeout=15)
        except Exception:
            self.proc.kill()
            self.proc.wait()
        samples = []
        for line in open(self.path):
            try:
                samples.append(json.loads(line))
            except ValueError:   # a line cut short by the termination
                pass
        for p in (self.path, self.path + ".go"):
            try:
                os.unlink(p)
            except OSError:
                pass
        return samples


def summarize_power(samples, t0, t1, launches):
    """The power record of a window [t0, t1] of ``launches`` back-to-back launches: medians of the
    readings taken in its middle half (the controller settles in the first quarter), the window's
    wall time per launch, and their product, the energy per launch."""
    import statistics
    lo, hi = t0 + (t1 - t0) / 4, t1 - (t1 - t0) / 4
    mid = [s for s in samples if "watts" in s and lo <= s["t"] <= hi]
    if not mid:
        errs = [s["error"] for s in samples if "error" in s]
        return {"error": errs[-1] if errs else "no amd-smi reading inside the window's middle half"}
    watts = statistics.median(s["watts"] for s in mid)
    mhz = statistics.median(s["mhz"] for s in mid)
    ms = (t1 - t0) * 1e3 / launches
    return {"watts": round(watts, 1), "cap_watts": POWER_CAP_W, "gfx_clock_mhz": int(round(mhz)),
            "ms_per_launch": round(ms, 4), "energy_per_launch_j": round(watts * ms * 1e-3, 3), "samples": len(mid),
            "seconds": round(t1 - t0, 2),
            "source": "live: amd-smi metric -p -c every 0.25 s beside launches back to back, medians over the "
                      "window's middle half"}


def power_window(launch, seconds, sampler):
    """Board power under ``launch`` (one step on torch's current stream, which is the null stream
    here, where the drop-in code object launches too), launched back to back for ``seconds`` with at
    most two chunks of 16 launches queued (an event per chunk), the sampler on meanwhile."""
    import torch
    from collections import deque
    for _ in range(4):
        launch()
    torch.cuda.synchronize()
    sampler.start()
    pending, n, t0 = deque(), 0, time.time()
    while True:
        for _ in range(16):
            launch()
        n += 16
        ev = torch.cuda.Event()
        ev.record()
        pending.append(ev)
        if len(pending) > 2:
            pending.popleft().synchronize()
        if time.time() - t0 >= seconds:
            break
    torch.cuda.synchronize()
    t1 = time.time()
    return summarize_power(sampler.stop(), t0, t1, n)


def read_power(label):
    """The board power and gfx clock measured under this workload (profiles/power_sites.txt: amd-smi
    sampled beside a long run of it), or None. Every large kernel here runs at the board's power
    cap, which is what holds the clock and with it roofline.frac. Not measured by this run."""
    rev = None
    try:
        for line in open(POWER_FILE):
            if line.startswith("kernel_revision:"):
                rev = line.split(":", 1)[1].strip()
            m = re.match(r"^  (\S.*?)\s{2,}([\d.]+)\s+(\d+)\s+([\d.]+)\s+([\d.]+)\s*$", line)
            if m and m.group(1) == label:
                return {"watts": float(m.group(2)), "cap_watts": POWER_CAP_W, "gfx_clock_mhz": int(m.group(3)),
                        "energy_per_launch_j": float(m.group(5)),
                        "source": f"profiles/power_sites.txt (amd-smi, kernel revision {rev or 'unrecorded'})"}
    except OSError:
        return None
    return None


def power_label(args):
    """The power_sites.txt row measured on this exact variant, or None."""
    if args.config == "gate_up_wgrad" and args.mfma == "k128":
        if args.out == "bf16" and args.lens == "multinomial":
            return "gate_up_wgrad, bf16 C"
        if args.out == "f32" and args.lens == "multinomial":
            return "gate_up_wgrad, fp32 C"
        if args.out == "f32_accum" and args.lens == "reference":
            return "gate_up_wgrad, fp32 accumulate (ref)"
    if args.config == "gate_up_fwd":
        if args.persistent_kernel in ("auto", "wide") and not args.row_align:
            return "gate_up_fwd, contiguous rows"
        if args.persistent_kernel in ("auto", "wide") and args.row_align == 128:
            return "gate_up_fwd, 128-byte rows"
        if args.persistent_kernel == "512" and not args.row_align:
            return "gate_up_fwd, 512-thread kernel"
    return None


def host_cores():
    """CPU cores this process may run on (its affinity set), the host share the CPU baseline has."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def print_info(pkg):
    """Resources of this build's code objects (the counterpart of the reference's kernel info
    printout, bench.py:544-589)."""
    from ggemm_asm_amd import harness
    for path in (pkg.CODE_OBJECT_PATH, *pkg.PERSISTENT_CODE_OBJECT_PATHS.values()):
        print(json.dumps(harness.kernel_info(path)), flush=True)


def fwd_operands(p, row_align):
    """A and B of a fwd / dgrad site, in buffers with row strides rounded up to row_align bytes
    (views of the logical shape) when row_align > 0."""
    import torch
    a, b = p.a, p.b
    if row_align and p.K % row_align:
        kp = -(-p.K // row_align) * row_align
        a = torch.zeros((p.M, kp), dtype=torch.uint8, device=p.a.device)[:, :p.K]
        a.copy_(p.a)
        b = torch.zeros((p.G, p.N, kp), dtype=torch.uint8, device=p.b.device)[:, :, :p.K]
        b.copy_(p.b)
    return a.view(p.a_dtype), b.view(torch.float8_e4m3fn)


def make_runner(pkg, p, dev, mfma, kernel="auto", row_align=0):
    """Closure launching one step of the workload; ``run.out`` is the output tensor it writes, so the
    last timed launch's result can be checked after timing."""
    import torch
    if hasattr(p, "a_format"):   # forward / data-gradient site: the persistent grouped GEMM
        sa = torch.tensor(p.a_scale, dtype=torch.float32, device=dev)
        sb = torch.tensor(p.b_scale, dtype=torch.float32, device=dev)
        out = torch.empty((p.M, p.N), dtype=torch.bfloat16, device=dev)
        a, b = fwd_operands(p, row_align)
        run = lambda: pkg.grouped_gemm_fp8_tensorwise(a, b, sa, sb, p.group_offs, out=out, kernel=kernel)
    elif p.is_mx:
        out = torch.empty((p.G, p.OUT_M, p.OUT_N), dtype=torch.bfloat16, device=dev)
        run = lambda: pkg.grouped_gemm_mxfp8_variable_k(p.lhs, p.rhs, p.lhs_mx, p.rhs_mx, p.group_offs, out=out)
    else:
        sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=dev)
        sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=dev)
        out = torch.empty((p.G, p.OUT_M, p.OUT_N), dtype=torch.bfloat16, device=dev)
        run = lambda: pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs, out=out,
                                                                  mfma=mfma)
    run.out = out
    return run


def time_steps(run, steps, warmup):
    import torch
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()          # the library launches on this stream
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info
        return max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        return os.cpu_count() or 1


PARITY_BAR = ("cos >= 0.99999 and max_rel <= 2e-2 over |ref| > 1e-3 * max|ref| of the whole output, no "
              "non-finite value, empty groups exactly zero")


def _bf16_bits(t):
    """Bit patterns (numpy uint16) of a bf16 tensor, or of an fp32 one rounded to bf16 (RNE)."""
    import numpy as np
    import torch
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _parity_record(orc, got_parts, refs, empty, groups):
    """The whole-output metrics of ``got_parts`` (one bf16-bit array per group, aligned with
    ``refs``) against the oracle, and whether they meet the bar."""
    import numpy as np
    amax = max((float(np.abs(orc.bf16_bits_to_f32(r)).max()) for r in refs if r.size), default=0.0)
    m = orc.compare_parts(zip(got_parts, refs), amax)
    m["empty_groups"] = len(empty)
    m["empty_zero"] = bool(all(np.all((got_parts[g] & 0x7FFF) == 0) for g in empty))
    m["groups"] = groups
    m["ok"] = bool(orc.parity_ok(m))
    m["bar"] = PARITY_BAR
    return {k: (round(v, 7) if isinstance(v, float) else v) for k, v in m.items()}


def oracle_leg(p, outs, seconds):
    """The numpy oracle over every group of the timed workload, run after the timed region.

    Parity: each group's oracle C (fp32 dequantize + per-group sgemm + bf16 RNE) against the C
    that the last timed launch left in each tensor of ``outs`` (name -> [G, OUT_M, OUT_N], bf16 or
    fp32 rounded to bf16), the whole tensor, every group: the reference checks the kernel it
    benchmarks in the same harness (reference bench.py:594-648; cosine over the whole output at
    :641-646). CPU baseline: the same oracle calls timed, over the groups computed until ~`seconds`
    of CPU time (the parity pass continues past it untimed); None when ``seconds`` <= 0.
    Returns ({name: parity record}, cpu_baseline)."""
    import numpy as np
    from oracle import vark_oracle as orc
    threads = _blas_threads()
    offs = p.group_offs.cpu().numpy()
    refs, empty = [], []
    done_flops, t_total, timed_groups, tokens = 0.0, 0.0, 0, 0
    for g in range(p.G):
        lo, hi = int(offs[g]), int(offs[g + 1])
        if hi == lo:
            refs.append(np.zeros((p.OUT_M, p.OUT_N), dtype=np.uint16))
            empty.append(g)
            continue
        L = p.lhs[lo:hi].cpu().numpy()
        R = p.rhs[lo:hi].cpu().numpy()
        sub = np.array([0, hi - lo], dtype=np.int64)
        t0 = time.perf_counter()
        if p.is_mx:   # MX groups start on 32-token blocks (groups padded to multiples of 32)
            ref = orc.vark_wgrad_mxfp8(L, R, p.lhs_mx[lo // 32:(hi + 31) // 32].cpu().numpy(),
                                       p.rhs_mx[lo // 32:(hi + 31) // 32].cpu().numpy(), sub)
        else:
            ref = orc.vark_wgrad_tensorwise(L, R, p.lhs_scale, p.rhs_scale, sub)
        dt = time.perf_counter() - t0
        refs.append(ref[0])
        if seconds > 0 and t_total < seconds:
            t_total += dt
            done_flops += 2.0 * (hi - lo) * p.OUT_M * p.OUT_N
            timed_groups += 1
            tokens += hi - lo
    parity = {name: _parity_record(orc, [_bf16_bits(out[g]) for g in range(p.G)], refs, empty,
                                   f"{p.G} of {p.G}")
              for name, out in outs.items()}
    base = None
    if timed_groups:
        base = {"value": round(done_flops / t_total / 1e12, 4), "unit": "TFLOPS", "cores": int(threads),
                "host_cores": host_cores(), "kind": "port",
                "sample": f"{timed_groups} of {p.G} groups ({tokens} tokens, {done_flops / 1e12:.2f} TFLOP) of "
                          f"{p.name}: numpy fp32 dequantize + OpenBLAS sgemm + bf16 RNE, {t_total:.1f} s"}
    return parity, base


def oracle_leg_fwd(p, outs, seconds):
    """``oracle_leg`` for a forward / data-gradient site: every row of every group of the output
    [M_total, N] each tensor of ``outs`` (name -> tensor) holds after the last timed launch against
    the persistent GEMM's oracle, and the CPU baseline from the same calls. Returns
    ({name: parity record}, cpu_baseline)."""
    import numpy as np
    from oracle import persistent_oracle as orp
    from oracle import vark_oracle as orc
    threads = _blas_threads()
    offs = p.group_offs.cpu().numpy()
    got = {name: _bf16_bits(out) for name, out in outs.items()}
    refs, parts, empty = [], {name: [] for name in outs}, []
    done_flops, t_total, timed_groups, rows = 0.0, 0.0, 0, 0
    for g in range(p.G):
        lo, hi = int(offs[g]), int(offs[g + 1])
        if hi == lo:
            continue
        A = p.a[lo:hi].cpu().numpy()
        B = p.b[g:g + 1].cpu().numpy()
        t0 = time.perf_counter()
        refs.append(orp.grouped_fp8(A, B, p.a_scale, p.b_scale, np.array([0, hi - lo], dtype=np.int64),
                                    p.a_format))
        dt = time.perf_counter() - t0
        for name in outs:
            parts[name].append(got[name][lo:hi])
        if seconds > 0 and t_total < seconds:
            t_total += dt
            done_flops += 2.0 * (hi - lo) * p.K * p.N
            timed_groups += 1
            rows += hi - lo
    parity = {name: _parity_record(orc, parts[name], refs, empty, f"{p.G} of {p.G} ({int(offs[-1] - offs[0])} rows)")
              for name in outs}
    base = None
    if timed_groups:
        base = {"value": round(done_flops / t_total / 1e12, 4), "unit": "TFLOPS", "cores": int(threads),
                "host_cores": host_cores(), "kind": "port",
                "sample": f"{timed_groups} of {p.G} groups ({rows} rows, {done_flops / 1e12:.2f} TFLOP) of "
                          f"{p.name}: numpy fp32 dequantize + OpenBLAS sgemm + bf16 RNE, {t_total:.1f} s"}
    return parity, base


def time_drop_in_co(pkg, p, dev, steps, warmup, power=None):
    """The drop-in code object (``variable_k_wgrad.co``) timed on the same inputs the way the
    reference times its own: loaded through the hipModule path, launched with the 16-entry
    kernelParams array on the null stream, grid num_cus x 512 threads, 64 KiB dynamic LDS
    (reference bench.py:364-413,768-801), HIP events on the null stream around ``steps``
    back-to-back launches. No C re-zeroing between launches: the kernel overwrites all of C.
    ``power``: a power window (``power_window`` bound to its duration and sampler) to run over the
    same launch afterwards, its record kept as ``power``. Returns (record, output tensor of the last
    launch)."""
    import torch
    from ggemm_asm_amd import harness
    module, func, name = harness.load_kernel(pkg.CODE_OBJECT_PATH)
    try:
        sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=dev)
        sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=dev)
        out = torch.empty((p.G, p.OUT_M, p.OUT_N), dtype=torch.bfloat16, device=dev)
        ncu = harness.get_num_cus(dev.index or 0)
        launch, _keep = harness.prepare_variable_k_args(func, p.lhs, p.rhs, out, sl, sr, p.group_offs, p.G, p.OUT_M,
                                                        p.OUT_N, ncu)
        torch.cuda.synchronize()
        ms = harness.time_null_stream(launch, steps, warmup)
        pw = power(launch) if power else None
    finally:
        harness.unload_kernel(module)
    geo = pkg.launch_geometry(p.OUT_N)
    rec = {"ms": round(ms, 4), "TFLOPS": round(p.flops / (ms * 1e-3) / 1e12, 2),
           "kernel": f"{os.path.basename(pkg.CODE_OBJECT_PATH)}: {name}, {geo['tile_m']}x{geo['tile_n']} tiles, "
                     f"grid {ncu} x {harness.BLOCK} threads, {harness.SHARED_MEM} B dynamic LDS, kernelParams launch "
                     f"on the null stream (what reference launcher.cpp / bench.py --kernel callers run)"}
    if pw:
        rec["power"] = pw
    return rec, out


def time_drop_in_co_fwd(pkg, p, dev, steps, warmup, row_align, power=None):
    """The persistent GEMM's drop-in code object for the site's A format
    (``persistent_e4m3.co`` / ``persistent_e5m2.co``, the 512-thread kernel) timed as
    ``time_drop_in_co`` times the wgrad's: the reference's hipModule path with the 16-entry
    kernelParams array on the null stream (reference bench.py:312-361), on the same operands (with
    ``row_align``, the same padded views); ``power`` as there. Returns (record, output tensor of the
    last launch)."""
    import torch
    from ggemm_asm_amd import harness
    path = pkg.PERSISTENT_CODE_OBJECT_PATHS[p.a_format]
    module, func, name = harness.load_kernel(path)
    try:
        sa = torch.tensor(p.a_scale, dtype=torch.float32, device=dev)
        sb = torch.tensor(p.b_scale, dtype=torch.float32, device=dev)
        a, b = fwd_operands(p, row_align)
        out = torch.empty((p.M, p.N), dtype=torch.bfloat16, device=dev)
        ncu = harness.get_num_cus(dev.index or 0)
        launch, _keep = harness.prepare_persistent_args(func, a, b, out, sa, sb, p.group_offs, p.G, p.N, p.K, ncu)
        torch.cuda.synchronize()
        ms = harness.time_null_stream(launch, steps, warmup)
        pw = power(launch) if power else None
    finally:
        harness.unload_kernel(module)
    geo = pkg.launch_geometry(p.N)
    rec = {"ms": round(ms, 4), "TFLOPS": round(p.flops / (ms * 1e-3) / 1e12, 2),
           "kernel": f"{os.path.basename(path)}: {name}, {geo['tile_m']}x{geo['tile_n']} tiles, grid {ncu} x "
                     f"{harness.BLOCK} threads, {harness.SHARED_MEM} B dynamic LDS, kernelParams launch on the null "
                     f"stream (what the reference's bench.py --kernel callers of this site run)"}
    if pw:
        rec["power"] = pw
    return rec, out


def quant_workload(pkg, name, seed, dev):
    """(runner, bytes per call, config dict, cpu-baseline callable) of a producer workload."""
    import torch
    gen = torch.Generator(device=dev).manual_seed(seed)
    H = 16
    hist, calls = None, [0]
    if name.endswith("_delayed"):
        # delayed scaling in steady state: a history of H entries, the slot cycling through it
        hist = torch.empty(H, dtype=torch.float32, device=dev)

        def slot():
            calls[0] += 1
            return calls[0] % H
    if name in ("quant_tensorwise", "quant_tensorwise_delayed"):
        x = torch.randn((pkg.inputs.M_TOTAL, pkg.inputs.F_DIM), generator=gen, device=dev, dtype=torch.bfloat16)
        n = x.numel()
        if hist is None:
            run = lambda: pkg.quantize_fp8_tensorwise(x, "e4m3")
            cfg = {"workload": name, "x": "bf16 [131072, 2880] (randn)", "out": "e4m3fn, fp32 scale + amax",
                   "bytes_per_element": "2 (amax pass) + 2 (quantize pass) + 1 (fp8 out)"}
            nbytes = 5 * n
        else:
            run = lambda: pkg.quantize_fp8_tensorwise_delayed(x, hist, slot(), "e4m3")
            cfg = {"workload": name, "x": "bf16 [131072, 2880] (randn)",
                   "out": f"e4m3fn, fp32 scale from an amax history of {H}, amax recorded in the pass",
                   "bytes_per_element": "2 (quantize pass, amax reduced in it) + 1 (fp8 out)"}
            nbytes = 3 * n
    elif name in ("quant_weight_transpose", "quant_weight_transpose_delayed"):
        E, F, F2 = pkg.inputs.E_EXPERTS, pkg.inputs.F_DIM, pkg.inputs.F2_DIM
        x = (torch.randn((E, F2, F), generator=gen, device=dev, dtype=torch.bfloat16) * 0.02)
        n = x.numel()
        if hist is None:
            run = lambda: pkg.quantize_fp8_tensorwise_transpose(x, "e4m3")
            cfg = {"workload": name, "x": "bf16 weight [32, 5760, 2880] (randn * 0.02)",
                   "out": "e4m3fn q [32, 5760, 2880] + q^T [32, 2880, 5760], fp32 scale + amax",
                   "bytes_per_element": "2 (amax pass) + 2 (quantize pass) + 1 (q) + 1 (q^T)"}
            nbytes = 6 * n
        else:
            run = lambda: pkg.quantize_fp8_tensorwise_transpose_delayed(x, hist, slot(), "e4m3")
            cfg = {"workload": name, "x": "bf16 weight [32, 5760, 2880] (randn * 0.02)",
                   "out": f"e4m3fn q [32, 5760, 2880] + q^T [32, 2880, 5760], fp32 scale from an amax history "
                          f"of {H}, amax recorded in the pass",
                   "bytes_per_element": "2 (quantize pass, amax reduced in it) + 1 (q) + 1 (q^T)"}
            nbytes = 4 * n
    else:
        lens = pkg.inputs.multinomial_lens(pkg.inputs.E_EXPERTS, pkg.inputs.M_TOTAL, torch.Generator().manual_seed(seed))
        offs = pkg.inputs.make_group_offs(lens).to(dev)
        x = torch.randn((pkg.inputs.M_TOTAL, pkg.inputs.F2_DIM), generator=gen, device=dev,
                        dtype=torch.bfloat16).mul_(1e-3)
        n = x.numel()
        run = lambda: pkg.quantize_mxfp8_grouped(x, offs, "e5m2")
        cfg = {"workload": name, "x": "bf16 [131072, 5760] (randn * 1e-3), 32 multinomial groups",
               "out": "e5m2 + e8m0 per 32-token block, groups padded to 32 rows",
               "bytes_per_element": "2 (read) + 1 (fp8 out) + 1/32 (e8m0)"}
        nbytes = n * (3 + 1 / 32)

    if hist is not None:
        hist.fill_(float(pkg.amax(x)))

    def cpu(seconds):
        """numpy oracle on row slices of the same tensor until ~`seconds`; GB/s of the same
        per-element byte count."""
        import numpy as np
        from oracle import quant_oracle as orq
        rows, t_total, done = 4096, 0.0, 0
        xc = x.reshape(-1, x.shape[-1])[:rows].float().cpu().numpy()
        h_np = hist.cpu().numpy() if hist is not None else None
        while t_total < seconds:
            t0 = time.perf_counter()
            if name == "quant_tensorwise":
                orq.quantize_tensorwise(xc, "e4m3")
            elif name == "quant_weight_transpose":
                np.ascontiguousarray(orq.quantize_tensorwise(xc, "e4m3")[0].T)
            elif name == "quant_tensorwise_delayed":
                orq.quantize_tensorwise_delayed(xc, h_np, 1, "e4m3")
            elif name == "quant_weight_transpose_delayed":
                np.ascontiguousarray(orq.quantize_tensorwise_delayed(xc, h_np, 1, "e4m3")[0].T)
            else:
                orq.quantize_mx_grouped(xc, np.array([0, rows], np.int64), "e5m2", out_rows=rows)
            t_total += time.perf_counter() - t0
            done += xc.size
        return {"value": round(done * (nbytes / n) / t_total / 1e9, 3), "unit": "GB/s", "cores": 1,
                "host_cores": host_cores(), "kind": "port",
                "sample": f"{done // xc.size} x {rows} rows of {name}'s input through the numpy oracle, "
                          f"{t_total:.1f} s"}

    return run, nbytes, cfg, cpu


def main_quant(args, pkg, dev):
    run, nbytes, cfg, cpu = quant_workload(pkg, args.config, args.seed, dev)
    ms = time_steps(run, args.steps, args.warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {"metric": f"GB/s of the FP8 quantization producer ({args.config}) on 1 MI355X", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16->fp8",
            "data": "synthetic", "config": cfg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic(args.config)[0],
                         "traffic_source": read_traffic(args.config)[1]},
            "cpu_baseline": cpu(args.cpu_seconds) if args.cpu_seconds > 0 else None}
    print(json.dumps(line), flush=True)


def main_layer(args, pkg, dev):
    import torch
    from ggemm_asm_amd.autograd import FP8DelayedScaling, grouped_linear_fp8
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    M, K, N, G = pkg.inputs.M_TOTAL, pkg.inputs.F_DIM, pkg.inputs.F2_DIM, pkg.inputs.E_EXPERTS
    offs = pkg.inputs.make_group_offs(pkg.inputs.make_group_lens_reference()).to(dev)
    x = torch.randn((M, K), generator=gen, device=dev, dtype=torch.bfloat16).requires_grad_(True)
    w = (torch.randn((G, N, K), generator=gen, device=dev, dtype=torch.bfloat16) * 0.02).requires_grad_(True)
    dy = torch.randn((M, N), generator=gen, device=dev, dtype=torch.bfloat16) * 1e-3
    main_grad = torch.zeros((G, K, N), dtype=torch.float32, device=dev)
    # delayed: the first (warm-up) step seeds the history with current scaling
    rec = FP8DelayedScaling(16) if args.scaling == "delayed" else None

    def step():
        x.grad = None
        out = grouped_linear_fp8(x, w, offs, main_grad=main_grad, scaling=rec)
        out.backward(dy)

    ms = time_steps(step, args.steps, args.warmup)
    flops = 3 * 2.0 * M * K * N
    tflops = flops / (ms * 1e-3) / 1e12
    extra = None
    if args.extra:
        # gradient accumulation: the weight is unchanged between micro-batches, so its fp8 copy
        # (and q^T) comes from the cache and the weight quantization pass drops out of the step
        from ggemm_asm_amd.autograd import FP8WeightCache
        cache = FP8WeightCache()

        def step_cached():
            x.grad = None
            out = grouped_linear_fp8(x, w, offs, main_grad=main_grad, weight_cache=cache, scaling=rec)
            out.backward(dy)

        t = time_steps(step_cached, max(args.steps // 2, 10), max(args.warmup // 2, 5))
        extra = {"gate_up_layer_cached_weight": {"ms": round(t, 4), "TFLOPS": round(flops / (t * 1e-3) / 1e12, 2),
                                                 "cache_hits": cache.hits, "cache_misses": cache.misses}}
    line = {"metric": "ms + TFLOPS of one FP8 grouped linear training step (gate_up shape) on 1 MI355X",
            "value": round(tflops, 2), "unit": "TFLOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp8", "data": "synthetic",
            "config": {"workload": "gate_up_layer", "G": G, "M_total": M, "K": K, "N": N,
                       "step": "quantize x, w (e4m3) + fwd GEMM + quantize dy (e5m2) + dgrad GEMM + wgrad GEMM "
                               "accumulated into an fp32 main-grad",
                       "scaling": args.scaling + (" (amax history 16)" if rec else " (amax pass per tensor)"),
                       "inputs": "seed-42 exponential group sizes, randn bf16, in HBM"},
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP8_DENSE_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / FP8_DENSE_PEAK_TFLOPS, 4), "traffic": None},
            "cpu_baseline": None}
    if extra:
        line["extra"] = extra
    print(json.dumps(line), flush=True)


def main_sites(args, pkg, dev):
    """The reference's multi-site run (bench.py:690-858): each call site in turn with the
    reference's input recipe (seed-42 exponential group lengths, randn bf16 cast to fp8, scales
    0.1), then its summary table (ms, TFLOPS, TFLOP and share of the total per site, and the total)
    on stderr. The JSON line carries the sum over the sites; each site's row also carries the parity of
    its last timed output against the oracle over every group (unless --no-parity)."""
    import torch
    names = SITE_GROUPS.get(args.site, (args.site,))
    rows = []
    for name in names:
        if name in FWD_SITES:
            p = pkg.inputs.make_fwd_problem(name, seed=args.seed, device=dev)
        else:
            p = pkg.inputs.make_wgrad_site_problem(name, seed=args.seed, device=dev)
        torch.cuda.synchronize()
        run = make_runner(pkg, p, dev, args.mfma, args.persistent_kernel, args.row_align)
        ms = time_steps(run, args.steps, args.warmup)
        row = {"site": name, "ms": round(ms, 4), "TFLOPS": round(p.flops / (ms * 1e-3) / 1e12, 2),
               "TFLOP": round(p.flops / 1e12, 4)}
        if args.parity:   # the site's last timed output against the oracle, every group
            leg = oracle_leg_fwd if name in FWD_SITES else oracle_leg
            m = leg(p, {"library": run.out}, 0.0)[0]["library"]
            row["parity"] = {k: m[k] for k in ("ok", "cos", "max_rel", "nonfinite", "empty_zero", "groups")}
        rows.append(row)
        print(f"  {name}: {ms:.4f} ms" + (f", parity {'ok' if row['parity']['ok'] else 'FAILED'} (max_rel "
                                          f"{row['parity']['max_rel']:.4f})" if args.parity else ""),
              file=sys.stderr, flush=True)
        del p, run
    total_ms = sum(r["ms"] for r in rows)
    total_tflop = sum(r["TFLOP"] for r in rows)
    tflops = total_tflop / (total_ms * 1e-3)
    bar = "=" * 64
    print(bar, file=sys.stderr)
    print(f"{'Site':<16s} {'ms':>9} {'TFLOPS':>9} {'TFLOP':>8} {'% total':>8}", file=sys.stderr)
    print("-" * 64, file=sys.stderr)
    for r in rows:
        print(f"{r['site']:<16s} {r['ms']:9.4f} {r['TFLOPS']:9.1f} {r['TFLOP']:8.3f} "
              f"{100 * r['ms'] / total_ms:7.1f}%", file=sys.stderr)
    print("-" * 64, file=sys.stderr)
    print(f"{'TOTAL':<16s} {total_ms:9.4f} {tflops:9.1f} {total_tflop:8.3f} {'100.0':>7s}%", file=sys.stderr)
    print(bar, file=sys.stderr, flush=True)
    line = {"metric": f"ms + TFLOPS (% FP8 peak) summed over the {args.site} call sites on 1 MI355X",
            "value": round(tflops, 2), "unit": "TFLOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(total_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp8", "data": "synthetic",
            "config": {"workload": args.site, "sites": rows,
                       "inputs": "reference recipe: seed-42 exponential group sizes, randn bf16 cast to fp8, "
                                 "scales 0.1, in HBM",
                       "step": "one launch of each site's grouped GEMM, sites run one after the other"},
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP8_DENSE_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / FP8_DENSE_PEAK_TFLOPS, 4), "traffic": None},
            "cpu_baseline": None}
    print(json.dumps(line), flush=True)
    bad = [r["site"] for r in rows if r.get("parity") and not r["parity"]["ok"]]
    if bad:
        print(f"bench.py: the output of {', '.join(bad)} fails the parity bar against the oracle ({PARITY_BAR})",
              file=sys.stderr, flush=True)
        sys.exit(1)


def main():
    args = parse_args()
    if args.power_sampler:
        power_sampler(args.power_sampler, args.power_interval)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the grouped wgrad needs no collective and this build runs "
              f"on a single MI355X (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    if args.power_seconds > 0 and (args.site or args.config in QUANT_CONFIGS + LAYER_CONFIGS or args.info
                                   or args.copy_calibration_mb):
        raise SystemExit("--power-seconds applies to the single-kernel configs")
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb, args.steps)
        return
    # the power sampler's child process starts here, before anything touches the GPU
    sampler = PowerSampler() if args.power_seconds > 0 else None
    try:
        run_bench(args, sampler)
    finally:
        if sampler is not None and sampler.proc.poll() is None:
            sampler.stop()


def run_bench(args, sampler):
    from __graft_entry__ import load_package
    pkg = load_package()
    if args.info:
        print_info(pkg)
        return
    import torch
    dev = torch.device("cuda:0")
    if args.site:
        main_sites(args, pkg, dev)
        return
    if args.config in QUANT_CONFIGS:
        main_quant(args, pkg, dev)
        return
    if args.scaling != "current" and args.config not in LAYER_CONFIGS:
        raise SystemExit("--scaling applies to gate_up_layer")
    if args.config in LAYER_CONFIGS:
        main_layer(args, pkg, dev)
        return
    fwd = args.config in FWD_SITES
    tw_wgrad = args.config in ("gate_up_wgrad", "down_wgrad", "gate_up_zipf")
    if (args.persistent_kernel != "auto" or args.row_align) and not fwd:
        raise SystemExit("--persistent-kernel / --row-align apply to the fwd / dgrad sites")
    if (args.out != "bf16" or args.lens != "multinomial") and not tw_wgrad:
        raise SystemExit("--out / --lens apply to the tensorwise wgrad configs (gate_up_wgrad, down_wgrad, "
                         "gate_up_zipf)")
    if args.config == "constant":
        p = pkg.inputs.constant_problem(device=dev)
    elif fwd:
        p = pkg.inputs.make_fwd_problem(args.config, seed=args.seed, device=dev)
    elif args.config in SHARD_CONFIGS:
        p = pkg.inputs.make_problem("gate_up_wgrad", seed=args.seed, device=dev, **SHARD_CONFIGS[args.config])
        p.name = args.config
    else:
        lens = pkg.inputs.make_group_lens_reference() if args.lens == "reference" else None
        p = pkg.inputs.make_problem(args.config, seed=args.seed, device=dev, lens=lens)
    torch.cuda.synchronize()
    if args.out != "bf16":
        sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=dev)
        sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=dev)
        c32 = torch.zeros((p.G, p.OUT_M, p.OUT_N), dtype=torch.float32, device=dev)
        run = lambda: pkg.grouped_gemm_fp8_tensorwise_variable_k(p.lhs, p.rhs, sl, sr, p.group_offs, out=c32,
                                                                  out_dtype=torch.float32,
                                                                  accumulate=args.out == "f32_accum")
        run.out = c32
    else:
        run = make_runner(pkg, p, dev, args.mfma, args.persistent_kernel, args.row_align)
    ms = time_steps(run, args.steps, args.warmup)
    tflops = p.flops / (ms * 1e-3) / 1e12
    drop_in_co = (args.drop_in and not p.is_mx if not fwd else args.drop_in) and args.out == "bf16" \
        and args.mfma == "k128" and args.config not in SHARD_CONFIGS
    if sampler is not None and args.power_of == "drop_in" and not drop_in_co:
        raise SystemExit("--power-of drop_in needs the drop-in code object leg (bf16 C, k128, not --no-drop-in)")
    power_live = power_window(run, args.power_seconds, sampler) if sampler and args.power_of == "library" else None
    co_power = ((lambda launch: power_window(launch, args.power_seconds, sampler))
                if sampler and args.power_of == "drop_in" else None)
    # traffic measured for this exact variant (profiles/traffic_<config>[_<out>][_reference_lens].txt)
    traffic, traffic_source = read_traffic(args.config + ("" if args.out == "bf16" else "_" + args.out)
                                           + ("" if args.lens == "multinomial" else "_reference_lens"))
    if fwd:
        geo = pkg.launch_geometry(p.N)
        stride = -(-p.K // args.row_align) * args.row_align if args.row_align else p.K
        kern = args.persistent_kernel
        if kern == "auto":
            kern = pkg.persistent.selected_kernel(p.N, p.K, stride, stride, p.N)
        config = {"workload": p.name, "G": p.G, "M_total": p.M, "K": p.K, "N": p.N,
                  "a": {"e4m3": "e4m3fn", "e5m2": "e5m2"}[p.a_format], "b": "e4m3fn [G, N, K] (trans_b)",
                  "out": "bf16", "acc": "fp32",
                  "inputs": "reference recipe: seed-42 exponential group sizes, randn bf16 cast to fp8, "
                            "scales 0.1, in HBM" + (f", A and B row strides {stride} bytes" if stride != p.K else ""),
                  "kernel": ("hip gfx950 persistent wide 256x320 tiles (256 threads, one wave per SIMD, generated "
                             "assembly), 128-K stages, mfma 32x32x64" if kern == "wide"
                             else "hip gfx950 persistent {tile_m}x{tile_n} tiles, 128-K stages, mfma k128".format(**geo)),
                  "baseline_number": "none published for this site"}
        vs_baseline = None
    else:
        config = {"workload": p.name, "G": p.G, "M_total": p.M, "OUT_M": p.OUT_M, "OUT_N": p.OUT_N,
                  "lhs": "e4m3fn", "rhs": "e5m2",
                  "out": {"bf16": "bf16", "f32": "fp32", "f32_accum": "fp32, accumulated in place (C += result)"}[
                      args.out],
                  "acc": "fp32",
                  "inputs": "seeded N(0,1) / N(0,1e-3) quantized per-tensor, {} group sizes, in HBM".format(
                      "the reference's seed-42 exponential" if args.lens == "reference" else
                      {"gate_up_zipf": "Zipf-skewed"}.get(p.name, "multinomial")),
                  "kernel": ("hip gfx950 persistent {}x{} tiles, 256-thread workgroups (one wave per SIMD, "
                             "hand-placed accumulators), mfma 32x32x64".format(
                                 *((320, 320) if pkg.bf16_kernel(p.OUT_M, p.OUT_N) == "wide320" else (256, 384)))
                             if args.mfma == "k128" and pkg.bf16_kernel(p.OUT_M, p.OUT_N) != "192-row"
                             and (not p.is_mx or pkg.bf16_kernel(p.OUT_M, p.OUT_N) == "wide320")
                             else "hip gfx950 persistent {tile_m}x{tile_n} tiles, mfma {mfma}".format(
                                 mfma=args.mfma, **pkg.launch_geometry(p.OUT_N))),
                  "baseline_number": ("reference optimized ASM 3.515 ms / 1237 TFLOPS (README.md:60)"
                                      if p.name == "gate_up_wgrad" else "none published for this workload")}
        if p.is_mx:
            config["scales"] = "e8m0 per 32 tokens per column (MX block scaling)"
        vs_baseline = (round(tflops / REF_OPT_ASM_TFLOPS, 4) if p.name == "gate_up_wgrad" and args.out == "bf16"
                       else None)
    variant = "".join(f" {k}={v}" for k, v, d in (("out", args.out, "bf16"), ("lens", args.lens, "multinomial"))
                      if v != d)
    line = {
        "metric": f"ms + TFLOPS (% FP8 peak) for {p.name}{variant} G={p.G} M={p.M} on 1 MI355X",
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": vs_baseline,
        "dtype": "fp8",
        "data": "synthetic",
        "config": config,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP8_DENSE_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / FP8_DENSE_PEAK_TFLOPS, 4), "traffic": traffic,
                     "traffic_source": traffic_source},
    }
    label = power_label(args)
    power = power_live or (read_power(label) if label else None)
    if power:
        line["roofline"]["power"] = power
    if args.extra:
        extra = {}
        for name in ("down_wgrad", "gate_up_zipf", "gate_up_mx", "constant", *FWD_SITES):
            if name == args.config:
                continue
            if name == "constant":
                q = pkg.inputs.constant_problem(device=dev)
            elif name in FWD_SITES:
                q = pkg.inputs.make_fwd_problem(name, seed=args.seed, device=dev)
            else:
                q = pkg.inputs.make_problem(name, seed=args.seed, device=dev)
            r = make_runner(pkg, q, dev, args.mfma)
            t = time_steps(r, max(args.steps // 4, 10), max(args.warmup // 4, 5))
            extra[name] = {"ms": round(t, 4), "TFLOPS": round(q.flops / (t * 1e-3) / 1e12, 2)}
            if name == "gate_up_mx":      # the 192-row MX kernel beside the wide one the library picks
                o = torch.empty((q.G, q.OUT_M, q.OUT_N), dtype=torch.bfloat16, device=dev)
                r = lambda: pkg.grouped_gemm_mxfp8_variable_k(q.lhs, q.rhs, q.lhs_mx, q.rhs_mx, q.group_offs, out=o,
                                                              tile_m=192)
                t = time_steps(r, max(args.steps // 4, 10), max(args.warmup // 4, 5))
                extra["gate_up_mx_192_row"] = {"ms": round(t, 4), "TFLOPS": round(q.flops / (t * 1e-3) / 1e12, 2)}
                del o
            del q, r
        if args.mfma == "k128" and args.config == "gate_up_wgrad":
            r = make_runner(pkg, p, dev, "k32")
            t = time_steps(r, max(args.steps // 4, 10), max(args.warmup // 4, 5))
            extra["gate_up_wgrad_k32_mfma"] = {"ms": round(t, 4), "TFLOPS": round(p.flops / (t * 1e-3) / 1e12, 2)}
            # fp32 epilogues: fp32 C, and fp32 main-grad accumulation (C += result)
            sl = torch.tensor(p.lhs_scale, dtype=torch.float32, device=dev)
            sr = torch.tensor(p.rhs_scale, dtype=torch.float32, device=dev)
            c32 = torch.zeros((p.G, p.OUT_M, p.OUT_N), dtype=torch.float32, device=dev)
            for name, acc in (("gate_up_wgrad_f32_out", False), ("gate_up_wgrad_f32_accum", True)):
                r = lambda acc=acc: pkg.grouped_gemm_fp8_tensorwise_variable_k(
                    p.lhs, p.rhs, sl, sr, p.group_offs, out=c32, out_dtype=torch.float32, accumulate=acc)
                t = time_steps(r, max(args.steps // 4, 10), max(args.warmup // 4, 5))
                extra[name] = {"ms": round(t, 4), "TFLOPS": round(p.flops / (t * 1e-3) / 1e12, 2)}
            # the accumulate at the reference's seed-42 exponential group lengths
            q = pkg.inputs.make_problem("gate_up_wgrad", seed=args.seed, device=dev,
                                        lens=pkg.inputs.make_group_lens_reference())
            r = lambda: pkg.grouped_gemm_fp8_tensorwise_variable_k(
                q.lhs, q.rhs, sl, sr, q.group_offs, out=c32, out_dtype=torch.float32, accumulate=True)
            t = time_steps(r, max(args.steps // 4, 10), max(args.warmup // 4, 5))
            extra["gate_up_reference_lens_f32_accum"] = {"ms": round(t, 4),
                                                         "TFLOPS": round(q.flops / (t * 1e-3) / 1e12, 2)}
            del c32, q
        line["extra"] = extra
    # the drop-in code object on the same inputs: what reference-side callers (launcher.cpp,
    # bench.py --kernel) get; its C is checked against the oracle beside the library's
    outs = {} if args.out == "f32_accum" else {"library": run.out}
    co_steps = args.drop_in_steps or args.steps
    if drop_in_co and fwd:
        line["drop_in_co"], outs["drop_in_co"] = time_drop_in_co_fwd(pkg, p, dev, co_steps, args.warmup,
                                                                     args.row_align, co_power)
    elif drop_in_co:
        line["drop_in_co"], outs["drop_in_co"] = time_drop_in_co(pkg, p, dev, co_steps, args.warmup, co_power)
    # outside the timed region: the oracle over every group of the timed inputs, checked against
    # the last timed launch's output, and timed as the CPU baseline
    failed = []
    if fwd or (args.parity and outs):
        if args.parity:
            par, base = (oracle_leg_fwd if fwd else oracle_leg)(p, outs, args.cpu_seconds)
        else:
            par, base = {}, (oracle_leg_fwd(p, {}, args.cpu_seconds)[1] if args.cpu_seconds > 0 else None)
        line["parity"] = par.pop("library", None)
        if "drop_in_co" in par:
            line["drop_in_co"]["parity"] = par["drop_in_co"]
        failed += [n for n, m in [("library", line["parity"]), ("drop_in_co", par.get("drop_in_co"))]
                   if m and not m["ok"]]
    else:
        line["parity"] = None
        base = oracle_leg(p, {}, args.cpu_seconds)[1] if args.cpu_seconds > 0 else None
    if args.parity and args.out == "f32_accum":
        line["parity_note"] = "not checked here: C accumulates over the timed launches (fp32 accumulate); " \
                              "tests/test_gpu_wide.py checks C0 + result bit for bit"
    line["cpu_baseline"] = base
    print(json.dumps(line), flush=True)
    if failed:
        print(f"bench.py: the output of {', '.join(failed)} fails the parity bar against the oracle "
              f"({PARITY_BAR})", file=sys.stderr, flush=True)
        sys.exit(1)


if __name__ == "__main__":
    main()
