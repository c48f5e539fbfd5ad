"""Seeded synthetic inputs for the variable-K grouped wgrad path.

Group-length recipes and quantizers for the five workload configurations the
path is measured on (plumbing G=4/M=512, down_wgrad, gate_up_wgrad, gate_up
with Zipf skew, gate_up MXFP8), plus a restatement of the reference's own
generator (reference bench.py:205-223: exponential lengths, seed 42, int64
cumsum offsets).

Tensors are produced on ``device`` with a ``torch.Generator`` of that device,
so the bench can build the 1.1 GB inputs directly in HBM; tests that need
CPU-reproducible bytes pass ``device="cpu"``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

E4M3_MAX = 448.0
E5M2_MAX = 57344.0

E_EXPERTS = 32          # reference bench.py:148
M_TOTAL = 131072        # reference bench.py:149
F_DIM = 2880            # reference bench.py:150
F2_DIM = 5760           # reference bench.py:151

# wgrad call sites (reference bench.py:182-193): OUT_M x OUT_N, dtypes e4m3 x e5m2
WGRAD_SITES = {
    "down_wgrad": (F_DIM, F_DIM),
    "gate_up_wgrad": (F_DIM, F2_DIM),
}


# ----------------------------------------------------------------------------- lengths

def make_group_lens_reference(E: int = E_EXPERTS, M_total: int = M_TOTAL, seed: int = 42) -> torch.Tensor:
    """Reference bench.py:205-212 on the CPU: exponential draws normalised to M_total."""
    rng = torch.Generator().manual_seed(seed)
    raw = torch.empty(E).exponential_(generator=rng)
    raw = raw / raw.sum() * M_total
    lens = raw.long()
    lens[-1] = M_total - lens[:-1].sum()
    if lens.sum() != M_total or not bool((lens > 0).all()):
        raise ValueError("reference length recipe produced an empty group")
    return lens


def make_group_offs(group_lens: torch.Tensor) -> torch.Tensor:
    """Reference bench.py:215-218: offs[0]=0, offs[1:]=cumsum(lens) as int64."""
    offs = torch.zeros(len(group_lens) + 1, dtype=torch.int64, device=group_lens.device)
    offs[1:] = torch.cumsum(group_lens.long(), dim=0)
    return offs


def multinomial_lens(G: int, M: int, gen: torch.Generator) -> torch.Tensor:
    """Uniform multinomial routing of M tokens over G experts (~M/G each)."""
    draws = torch.multinomial(torch.ones(G), M, replacement=True, generator=gen)
    return torch.bincount(draws, minlength=G).long()


def zipf_lens(G: int, M: int, gen: torch.Generator, s: float = 1.2, n_empty: int = 4,
              n_tiny: int = 8) -> torch.Tensor:
    """Skewed routing: n_empty forced-empty experts, n_tiny experts of U[1,31] tokens, the rest
    proportional to rank^-s, scaled to sum to M (rounding residue on the largest), then a
    seeded shuffle of expert order."""
    n_zipf = G - n_empty - n_tiny
    if n_zipf < 1:
        raise ValueError("need at least one Zipf expert")
    tiny = torch.randint(1, 32, (n_tiny,), generator=gen).long()
    rest = M - int(tiny.sum())
    w = torch.arange(1, n_zipf + 1, dtype=torch.float64) ** (-s)
    z = torch.floor(w / w.sum() * rest).long()
    z[0] += rest - int(z.sum())
    lens = torch.cat([torch.zeros(n_empty, dtype=torch.long), tiny, z])
    perm = torch.randperm(G, generator=gen)
    return lens[perm]


def mx_lens(G: int, M: int, gen: torch.Generator, block: int = 32) -> torch.Tensor:
    """Multinomial lengths rounded to multiples of ``block`` with the total kept at M."""
    if M % block:
        raise ValueError("M must be a multiple of the MX block")
    lens = multinomial_lens(G, M, gen)
    r = torch.round(lens.double() / block).long() * block
    r[torch.argmax(r)] += M - int(r.sum())
    if bool((r < 0).any()):
        raise ValueError("rounding produced a negative group")
    return r


# ----------------------------------------------------------------------------- quantizers

def quantize_tensorwise(x: torch.Tensor, fmt: str) -> tuple[torch.Tensor, float]:
    """Per-tensor scale amax/fmax; saturating cast. Returns (uint8 bytes, fp32 scale)."""
    fmax = E4M3_MAX if fmt == "e4m3" else E5M2_MAX
    dt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    amax = float(x.abs().max())
    scale = float(torch.tensor(amax / fmax if amax > 0 else 1.0, dtype=torch.float32))
    q = (x / scale).clamp_(-fmax, fmax).to(dt)
    return q.view(torch.uint8), scale


def quantize_mx(x: torch.Tensor, fmt: str, block: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """OCP-MX style block scaling along dim 0 (tokens).

    e8m0 exponent X = floor(log2(fl32(amax_blk / fmax))) per ``block`` rows per column, clamped to
    [-127, 127] and stored as X+127; an all-zero block stores 127. Elements are divided by 2^X and
    saturate-clamped to +-fmax before the cast (block max lands in [fmax, 2 fmax)).
    Rows must be a multiple of ``block``. Returns (uint8 data [M, N], uint8 scales [M/block, N]).
    """
    fmax = E4M3_MAX if fmt == "e4m3" else E5M2_MAX
    dt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    M, N = x.shape
    if M % block:
        raise ValueError("rows must be a multiple of the block")
    xb = x.view(M // block, block, N)
    amax = xb.abs().amax(dim=1)
    X = torch.zeros_like(amax, dtype=torch.int32)
    nz = amax > 0
    # floor(log2(y)) taken exactly on the fp32 quotient y: frexp gives y = m 2^e, m in [0.5, 1)
    X[nz] = torch.frexp(amax[nz] / fmax).exponent.to(torch.int32) - 1
    X = X.clamp_(-127, 127)
    scale = torch.pow(2.0, X.to(torch.float32))
    q = (xb / scale.unsqueeze(1)).clamp_(-fmax, fmax).to(dt).view(M, N)
    return q.view(torch.uint8), (X + 127).to(torch.uint8)


# ----------------------------------------------------------------------------- configs

@dataclass
class VarKProblem:
    name: str
    lhs: torch.Tensor            # uint8 e4m3fn [M, OUT_M]
    rhs: torch.Tensor            # uint8 e5m2  [M, OUT_N]
    group_offs: torch.Tensor     # int64 [G+1]
    G: int
    OUT_M: int
    OUT_N: int
    lhs_scale: float = 1.0       # tensorwise scales (fp32)
    rhs_scale: float = 1.0
    lhs_mx: torch.Tensor | None = None   # uint8 e8m0 [M/32, OUT_M]
    rhs_mx: torch.Tensor | None = None   # uint8 e8m0 [M/32, OUT_N]
    meta: dict = field(default_factory=dict)

    @property
    def M(self) -> int:
        return int(self.lhs.shape[0])

    @property
    def flops(self) -> float:
        return 2.0 * self.M * self.OUT_M * self.OUT_N

    @property
    def is_mx(self) -> bool:
        return self.lhs_mx is not None


CONFIGS = ("plumbing", "down_wgrad", "gate_up_wgrad", "gate_up_zipf", "gate_up_mx")


def _randn(shape, std, gen, device):
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).mul_(std)


def make_problem(name: str, seed: int = 0, device: str | torch.device = "cpu", G: int | None = None,
                 M: int | None = None, OUT_M: int | None = None, OUT_N: int | None = None,
                 lens: torch.Tensor | None = None) -> VarKProblem:
    """Build one of the named configurations (optionally overriding sizes for scaled-down tests).

    Lengths always come from a CPU generator seeded ``seed`` (so offsets are identical on every
    device); values come from a generator on ``device`` seeded ``seed + 1``.
    """
    device = torch.device(device)
    cpu_gen = torch.Generator().manual_seed(seed)
    if name == "plumbing":
        G_, M_, om, on = 4, 512, 64, 128
        lens_ = torch.tensor([96, 160, 0, 256], dtype=torch.long)
    elif name in ("down_wgrad", "gate_up_wgrad", "gate_up_zipf", "gate_up_mx"):
        site = "down_wgrad" if name == "down_wgrad" else "gate_up_wgrad"
        om, on = WGRAD_SITES[site]
        G_, M_ = E_EXPERTS, M_TOTAL
        lens_ = None
    else:
        raise ValueError(f"unknown config {name!r}; choose from {CONFIGS}")
    G_ = G if G is not None else G_
    M_ = M if M is not None else M_
    om = OUT_M if OUT_M is not None else om
    on = OUT_N if OUT_N is not None else on
    if lens is not None:
        lens_ = torch.as_tensor(lens, dtype=torch.long)
    elif lens_ is None or G is not None or M is not None:
        if name == "gate_up_zipf":
            lens_ = zipf_lens(G_, M_, cpu_gen, n_empty=min(4, max(G_ - 2, 0)), n_tiny=min(8, max(G_ - 5, 0)))
        elif name == "gate_up_mx":
            lens_ = mx_lens(G_, M_, cpu_gen)
        else:
            lens_ = multinomial_lens(G_, M_, cpu_gen)
    if int(lens_.sum()) != M_ or len(lens_) != G_:
        raise ValueError("group lengths must sum to M and have G entries")
    offs = make_group_offs(lens_).to(device)

    gen = torch.Generator(device=device).manual_seed(seed + 1)
    x = _randn((M_, om), 1.0, gen, device)
    dy = _randn((M_, on), 1e-3, gen, device)
    meta = {"seed": seed, "lens": lens_.tolist()}
    if name == "gate_up_mx":
        ql, sl = quantize_mx(x, "e4m3")
        del x
        qr, sr = quantize_mx(dy, "e5m2")
        del dy
        return VarKProblem(name, ql, qr, offs, G_, om, on, lhs_mx=sl, rhs_mx=sr, meta=meta)
    ql, sl = quantize_tensorwise(x, "e4m3")
    del x
    qr, sr = quantize_tensorwise(dy, "e5m2")
    del dy
    return VarKProblem(name, ql, qr, offs, G_, om, on, lhs_scale=sl, rhs_scale=sr, meta=meta)


def constant_problem(G: int = 32, M: int = M_TOTAL, OUT_M: int = F_DIM, OUT_N: int = F2_DIM,
                     device: str | torch.device = "cpu") -> VarKProblem:
    """The reference launcher's timing inputs (launcher.cpp:97-112): bytes 0x38 everywhere
    (1.0 as e4m3fn, 0.5 as e5m2), scales 0.1, uniform split offs[i] = M*i/G."""
    lhs = torch.full((M, OUT_M), 0x38, dtype=torch.uint8, device=device)
    rhs = torch.full((M, OUT_N), 0x38, dtype=torch.uint8, device=device)
    offs = torch.tensor([M * i // G for i in range(G + 1)], dtype=torch.int64, device=device)
    return VarKProblem("constant", lhs, rhs, offs, G, OUT_M, OUT_N, lhs_scale=0.1, rhs_scale=0.1)


def make_wgrad_site_problem(name: str, seed: int = 42, device: str | torch.device = "cpu",
                            lens: torch.Tensor | None = None) -> VarKProblem:
    """A wgrad call site with the reference's own input recipe (reference bench.py:182-193,
    205-223, 731-737): seed-42 exponential group lengths over 32 experts and 131072 tokens, LHS and
    RHS torch.randn in bf16 cast straight to e4m3fn / e5m2 (no scaling), scales 0.1. ``seed``
    seeds the values (a generator on ``device``)."""
    if name not in WGRAD_SITES:
        raise ValueError(f"unknown site {name!r}; choose from {tuple(WGRAD_SITES)}")
    device = torch.device(device)
    om, on = WGRAD_SITES[name]
    lens_ = torch.as_tensor(lens, dtype=torch.long) if lens is not None else make_group_lens_reference()
    offs = make_group_offs(lens_).to(device)
    M_, G_ = int(lens_.sum()), len(lens_)
    gen = torch.Generator(device=device).manual_seed(seed)
    lhs = torch.randn((M_, om), generator=gen, device=device, dtype=torch.bfloat16).to(torch.float8_e4m3fn)
    rhs = torch.randn((M_, on), generator=gen, device=device, dtype=torch.bfloat16).to(torch.float8_e5m2)
    return VarKProblem(name, lhs.view(torch.uint8), rhs.view(torch.uint8), offs, G_, om, on, lhs_scale=0.1,
                       rhs_scale=0.1, meta={"seed": seed, "lens": lens_.tolist(), "recipe": "reference"})


# ----------------------------------------------------------------------------- fwd / dgrad sites

# persistent-kernel call sites (reference bench.py:153-180): K, N, A format (B is always e4m3fn,
# stored [G, N, K] -- trans_b=True)
FWD_SITES = {
    "gate_up_fwd": (F_DIM, F2_DIM, "e4m3"),
    "down_fwd": (F_DIM, F_DIM, "e4m3"),
    "down_dgrad": (F_DIM, F_DIM, "e5m2"),
    "gate_up_dgrad": (F2_DIM, F_DIM, "e5m2"),
}


@dataclass
class FwdProblem:
    name: str
    a: torch.Tensor              # uint8 [M, K] in a_format
    b: torch.Tensor              # uint8 e4m3fn [G, N, K]
    a_format: str                # "e4m3" | "e5m2"
    group_offs: torch.Tensor     # int64 [G+1]
    a_scale: float = 0.1
    b_scale: float = 0.1
    meta: dict = field(default_factory=dict)

    @property
    def M(self) -> int:
        return int(self.a.shape[0])

    @property
    def K(self) -> int:
        return int(self.a.shape[1])

    @property
    def N(self) -> int:
        return int(self.b.shape[1])

    @property
    def G(self) -> int:
        return int(self.b.shape[0])

    @property
    def flops(self) -> float:
        return 2.0 * self.M * self.K * self.N

    @property
    def a_dtype(self) -> torch.dtype:
        return torch.float8_e4m3fn if self.a_format == "e4m3" else torch.float8_e5m2


def make_fwd_problem(name: str, seed: int = 0, device: str | torch.device = "cpu",
                     lens: torch.Tensor | None = None, K: int | None = None, N: int | None = None) -> FwdProblem:
    """A call site of the persistent kernel with the reference's own input recipe (reference
    bench.py:205-223,238-247): seed-42 exponential group lengths over 32 experts and 131072 rows,
    values torch.randn in bf16 cast straight to fp8 (no scaling), scales 0.1. ``seed`` seeds the
    values (a generator on ``device``); ``lens``/``K``/``N`` override sizes for scaled-down tests."""
    if name not in FWD_SITES:
        raise ValueError(f"unknown site {name!r}; choose from {tuple(FWD_SITES)}")
    device = torch.device(device)
    K_, N_, fmt = FWD_SITES[name]
    K_ = K if K is not None else K_
    N_ = N if N is not None else N_
    lens_ = torch.as_tensor(lens, dtype=torch.long) if lens is not None else make_group_lens_reference()
    offs = make_group_offs(lens_).to(device)
    M_, G_ = int(lens_.sum()), len(lens_)
    gen = torch.Generator(device=device).manual_seed(seed)
    adt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    a = torch.randn((M_, K_), generator=gen, device=device, dtype=torch.bfloat16).to(adt).view(torch.uint8)
    b = torch.randn((G_, N_, K_), generator=gen, device=device, dtype=torch.bfloat16).to(torch.float8_e4m3fn)
    return FwdProblem(name, a, b.view(torch.uint8), fmt, offs, meta={"seed": seed, "lens": lens_.tolist()})
