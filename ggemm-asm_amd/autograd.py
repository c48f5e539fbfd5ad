"""Autograd op for an FP8 grouped linear layer (MoE experts) built on the three kernels.

``grouped_linear_fp8(x, w, group_offs)`` computes ``out[r] = x[r] @ w[g]^T`` for the rows ``r`` of
group ``g`` (``offs[g] <= r < offs[g+1]``) in FP8 with per-tensor scales, and its backward. It is
the caller the reference's kernels serve: the reference harness runs the three GEMMs of this layer
separately (reference bench.py:153-193: gate_up_fwd / down_fwd ``x @ W^T``, down_dgrad /
gate_up_dgrad ``dy @ W``, down_wgrad / gate_up_wgrad ``dW = x^T @ dy``), with the quantization and
the autograd wiring left to the framework (Primus-Turbo, not vendored).

* forward: x -> e4m3 and w -> e4m3 (per-tensor amax scales, the quantization producer; when x
  needs a gradient the weight pass also writes qw^T [G, K, N], the data-gradient GEMM's B); every
  fp8 operand is written with rows starting on 128-byte lines (padded row stride);
  ``out = grouped_gemm_fp8_tensorwise(qx, qw, sx, sw, offs)`` (persistent kernel), bf16; rows
  past offs[G] (tokens the routing dropped) are zero in out and in dx.
  Saved for backward: the fp8 tensors and their scales (1 byte per element, not the bf16 inputs).
* backward: dy -> e5m2;
  ``dx[r] = dy[r] @ w[g]`` — the persistent kernel with B = qw^T (K-major [G, N_out=K, K_red=N],
  written by the forward's quantization pass); ``dW[g] = dy_g^T @ x_g`` — the
  variable-K kernel computes ``x_g^T @ dy_g`` (the reference's wgrad orientation: e4m3 LHS, e5m2
  RHS, C [G, K, N]) and the gradient is its transpose ([G, N, K], a view). With
  ``main_grad=`` an fp32 [G, K, N] tensor, dW is accumulated into it instead (the fp32 epilogue,
  beta = 1) and the returned weight gradient is None.
* ``weight_cache=FP8WeightCache()``: the weight's quantization (qw, qw^T, scale) is kept between
  calls and redone only when the weight changes (its storage, shape or version counter, which an
  in-place write through the weight tensor bumps; writes through ``.data`` or raw pointers do not,
  so ``cache.attach(optimizer)`` or ``cache.invalidate()`` covers those). With gradient
  accumulation over several micro-batches the weight pass then runs once per update instead of
  once per step.
* ``scaling=FP8DelayedScaling()``: x, w and dy are quantized with delayed scaling (the largest
  amax of their previous calls, recorded on the device in the quantizing pass itself), which drops
  the standalone amax passes; values beyond the historical range saturate at +-fmax.
There is no CPU path: the tensors must live on a gfx950 GPU.
"""
from __future__ import annotations

import weakref

import torch

from .persistent import grouped_gemm_fp8_tensorwise
from .quant import (quantize_fp8_tensorwise, quantize_fp8_tensorwise_delayed, quantize_fp8_tensorwise_transpose,
                    quantize_fp8_tensorwise_transpose_delayed)
from .vark import grouped_gemm_fp8_tensorwise_variable_k

_LINE = 128   # bytes per cache line


def _quantize_weight(w, with_transpose, scaling=None):
    """(qw, qw^T or None, scale) of a [G, N, K] weight, rows on 128-byte lines; with ``scaling``
    (an FP8DelayedScaling) by its delayed recipe for the role "w"."""
    if scaling is not None:
        return scaling.quantize_weight(w.contiguous(), with_transpose)
    if with_transpose:
        qw, qwt, sw, _ = quantize_fp8_tensorwise_transpose(w.contiguous(), "e4m3", row_align=_LINE)
        return qw, qwt, sw
    qw, sw, _ = quantize_fp8_tensorwise(w.contiguous(), "e4m3", row_align=_LINE)
    return qw, None, sw


class FP8WeightCache:
    """One weight's e4m3 quantization, kept while the weight is unchanged.

    An entry is reused only for the same tensor object (held by a weak reference, so a new tensor
    that happens to reuse the old one's memory never hits) with the same storage address, shape,
    strides, dtype and version counter. An in-place write through the weight itself (``copy_``,
    ``add_``, an optimizer that updates the parameter tensor in place) bumps the version and the
    next call quantizes again. Writes that bypass the version counter are NOT seen: through
    ``w.data`` (a separate tensor with its own counter), through a raw pointer (fused multi-tensor
    optimizer kernels, C extensions), or from another process. For those, call ``invalidate()``
    after the update, or ``attach(optimizer)`` once, which invalidates after every
    ``optimizer.step()``. A cached entry without q^T is upgraded when a call needs the data
    gradient. ``hits`` / ``misses`` count lookups."""

    def __init__(self):
        self._ref = None
        self._key = None
        self._val = None
        self.hits = 0
        self.misses = 0

    @staticmethod
    def _key_of(w):
        return (w.data_ptr(), tuple(w.shape), tuple(w.stride()), w.dtype, str(w.device), w._version)

    def get(self, w, with_transpose, scaling=None):
        key = self._key_of(w)
        same = self._ref is not None and self._ref() is w and self._key == key
        if same and (self._val[1] is not None or not with_transpose):
            self.hits += 1
            return self._val
        self.misses += 1
        self._val = _quantize_weight(w, with_transpose, scaling)
        self._ref, self._key = weakref.ref(w), key
        return self._val

    def invalidate(self):
        """Drop the entry: the next call quantizes the weight again."""
        self._ref = self._key = self._val = None

    clear = invalidate

    def attach(self, optimizer):
        """Invalidate after every ``optimizer.step()`` (a torch.optim post-step hook), whatever
        path the optimizer writes the weight through. Returns the hook's handle."""
        return optimizer.register_step_post_hook(lambda *_: self.invalidate())


class FP8DelayedScaling:
    """Delayed-scaling recipe for one layer's activations (``"x"``, forward), weight (``"w"``,
    forward; with a weight cache only on its misses) and output gradients (``"dy"``, backward).

    Each tensor role keeps an fp32 amax history of ``history_len`` entries and the slot of its last
    call (an int32), both on the device. The first call for a role quantizes with the tensor's own
    amax (current scaling) and records it in slot 0; every later call advances the slot on the
    device to (slot + 1) % history_len, scales by the largest amax in the other slots, i.e. of up
    to ``history_len - 1`` previous calls, and writes this tensor's amax into the slot in the same
    pass. The amax pass over the tensor is gone; a tensor whose values outgrow the history
    saturates at +-fmax for that call. Because the slot advances on the device, a HIP graph that
    captures the layer rolls through the history on every replay; the first call of each role
    (the seeding one) must run eagerly, before any capture. ``calls`` counts the calls per role
    made from Python (a graph replay does not pass through here)."""

    def __init__(self, history_len: int = 16):
        if not 2 <= history_len <= 1024:
            raise ValueError("history_len must be in [2, 1024]")
        self.history_len = history_len
        self.history: dict[str, torch.Tensor] = {}
        self.slot: dict[str, torch.Tensor] = {}
        self.calls: dict[str, int] = {}

    def _state(self, role: str, device):
        """(history, device slot) of this role, or (None, None) before its first call on ``device``."""
        hist = self.history.get(role)
        if hist is None or hist.device != device:
            return None, None
        return hist, self.slot[role]

    def _seed(self, role: str, am: torch.Tensor):
        hist = torch.zeros(self.history_len, dtype=torch.float32, device=am.device)
        hist[:1].copy_(am.reshape(1))
        self.history[role] = hist
        self.slot[role] = torch.zeros(1, dtype=torch.int32, device=am.device)
        self.calls[role] = 1

    @staticmethod
    def _no_seed_in_capture(role: str):
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"FP8DelayedScaling: the first call for {role!r} seeds its amax history with current "
                               "scaling and must run eagerly; run one step before capturing a graph")

    def quantize(self, role: str, x: torch.Tensor, fmt: str):
        """(q, scale) of x for this role, rows on 128-byte lines."""
        hist, slot = self._state(role, x.device)
        if hist is None:
            self._no_seed_in_capture(role)
            q, scale, am = quantize_fp8_tensorwise(x, fmt, row_align=_LINE)
            self._seed(role, am)
            return q, scale
        q, scale = quantize_fp8_tensorwise_delayed(x, hist, slot, fmt, row_align=_LINE)
        self.calls[role] += 1
        return q, scale

    def quantize_weight(self, w: torch.Tensor, with_transpose: bool):
        """(qw, qw^T or None, scale) of a contiguous [G, N, K] weight (e4m3) for the role "w"."""
        if not with_transpose:
            q, scale = self.quantize("w", w, "e4m3")
            return q, None, scale
        hist, slot = self._state("w", w.device)
        if hist is None:
            self._no_seed_in_capture("w")
            qw, qwt, scale, am = quantize_fp8_tensorwise_transpose(w, "e4m3", row_align=_LINE)
            self._seed("w", am)
            return qw, qwt, scale
        qw, qwt, scale = quantize_fp8_tensorwise_transpose_delayed(w, hist, slot, "e4m3", row_align=_LINE)
        self.calls["w"] += 1
        return qw, qwt, scale


class GroupedLinearFP8(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, group_offs, main_grad, weight_cache=None, scaling=None):
        if x.dim() != 2 or w.dim() != 3 or x.shape[1] != w.shape[2]:
            raise ValueError("x must be [M, K] and w [G, N, K]")
        if w.shape[0] != group_offs.numel() - 1:
            raise ValueError("w holds one weight per group")
        # operand rows start on 128-byte lines (padded buffers): K-major rows of K = 2880 bytes
        # would otherwise straddle lines and cost the GEMMs 1.5 line requests per row segment
        if scaling is not None:
            qx, sx = scaling.quantize("x", x.contiguous(), "e4m3")
        else:
            qx, sx, _ = quantize_fp8_tensorwise(x.contiguous(), "e4m3", row_align=_LINE)
        if weight_cache is not None:
            qw, qwt, sw = weight_cache.get(w, ctx.needs_input_grad[0], scaling)
        else:
            qw, qwt, sw = _quantize_weight(w, ctx.needs_input_grad[0], scaling)
        # rows past offs[G] (tokens the routing dropped) come out as exact zeros
        out = grouped_gemm_fp8_tensorwise(qx, qw, sx, sw, group_offs, zero_tail=True)
        ctx.save_for_backward(qx, sx, qwt, sw, group_offs)
        ctx.main_grad = main_grad
        ctx.scaling = scaling
        ctx.x_dtype, ctx.w_dtype = x.dtype, w.dtype
        return out

    @staticmethod
    def backward(ctx, dy):
        qx, sx, qwt, sw, group_offs = ctx.saved_tensors
        if ctx.scaling is not None:
            qdy, sdy = ctx.scaling.quantize("dy", dy.contiguous(), "e5m2")
        else:
            qdy, sdy, _ = quantize_fp8_tensorwise(dy.contiguous(), "e5m2", row_align=_LINE)
        dx = dw = None
        if ctx.needs_input_grad[0]:
            # dx[r] = dy[r] @ w[g]: B[g] = w[g]^T, [N_out = K, K_red = N] K-major
            dx = grouped_gemm_fp8_tensorwise(qdy, qwt, sdy, sw, group_offs, zero_tail=True)
            dx = dx.to(ctx.x_dtype)
        if ctx.needs_input_grad[1] or ctx.main_grad is not None:
            if ctx.main_grad is not None:
                grouped_gemm_fp8_tensorwise_variable_k(qx, qdy, sx, sdy, group_offs, out=ctx.main_grad,
                                                       accumulate=True)
            else:
                dwt = grouped_gemm_fp8_tensorwise_variable_k(qx, qdy, sx, sdy, group_offs)   # [G, K, N]
                dw = dwt.transpose(1, 2).to(ctx.w_dtype)
        return dx, dw, None, None, None, None


def grouped_linear_fp8(x: torch.Tensor, w: torch.Tensor, group_offs: torch.Tensor,
                       main_grad: torch.Tensor | None = None,
                       weight_cache: FP8WeightCache | None = None,
                       scaling: FP8DelayedScaling | None = None) -> torch.Tensor:
    """FP8 grouped linear layer: ``out[r] = x[r] @ w[g]^T`` for the rows of group g, bf16 out.

    x: bf16 / fp32 [M, K] (rows grouped by expert); w: bf16 / fp32 [G, N, K]; group_offs: int64
    [G+1] on the device. Backward gives dx [M, K] and dw [G, N, K]; with ``main_grad`` (fp32
    [G, K, N], the wgrad kernel's orientation) the weight gradient is added into it instead. With
    ``weight_cache`` the weight's fp8 copy is reused while the weight is unchanged. With ``scaling``
    (one FP8DelayedScaling per layer) x, w and dy take delayed scaling (module docstring)."""
    if main_grad is not None:
        if main_grad.dtype != torch.float32 or tuple(main_grad.shape) != (w.shape[0], w.shape[2], w.shape[1]):
            raise ValueError(f"main_grad must be fp32 [G, K, N] = {[w.shape[0], w.shape[2], w.shape[1]]}")
    return GroupedLinearFP8.apply(x, w, group_offs, main_grad, weight_cache, scaling)
