"""GPU checks of the FP8 grouped linear autograd op (forward, dgrad, wgrad through the C ABI).

Each output is compared with the oracle composition on the same fp8 bytes (the producer is
deterministic, so the test re-quantizes the inputs to obtain them), to the bar's tolerance; and
with an unquantized float64 reference of the layer, which only fp8 quantization separates from it
(cosine >= 0.99) -- a check of the wiring (orientations, transposes, scales), not of the kernels.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _bytes(t):
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def _cos(a, b):
    a, b = a.detach().double().ravel(), b.detach().double().ravel()
    return float(a @ b / (a.norm() * b.norm() + 1e-300))


@pytest.mark.parametrize("lens,K,N", [([100, 0, 257, 31, 64], 256, 384), ([600, 300], 2880 // 9, 640)])
def test_grouped_linear_fp8_fwd_bwd(pkg, orc, orp, cuda, lens, K, N):
    from ggemm_asm_amd.autograd import grouped_linear_fp8
    g = torch.Generator().manual_seed(K + N)
    G, M = len(lens), sum(lens)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(cuda).requires_grad_(True)
    w = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16).to(cuda).requires_grad_(True)
    dy = (torch.randn((M, N), generator=g) * 1e-2).to(torch.bfloat16).to(cuda)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    _say(f"grouped linear fp8 lens={lens} K={K} N={N}")
    out = grouped_linear_fp8(x, w, offs)
    out.backward(dy)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and x.grad.shape == x.shape and w.grad.shape == w.shape
    o = offs.cpu().numpy()

    # the same fp8 bytes the op used
    qx, sx, _ = pkg.quantize_fp8_tensorwise(x.detach(), "e4m3")
    qw, sw, _ = pkg.quantize_fp8_tensorwise(w.detach(), "e4m3")
    qdy, sdy, _ = pkg.quantize_fp8_tensorwise(dy, "e5m2")
    sx, sw, sdy = float(sx), float(sw), float(sdy)
    ref_out = orp.grouped_fp8(_bytes(qx), _bytes(qw), sx, sw, o, "e4m3")
    m = orc.compare(pkg.as_bf16_bits(out), ref_out)
    _say(f"forward: {m}")
    assert orc.parity_ok(m)
    ref_dx = orp.grouped_fp8(_bytes(qdy), _bytes(qw), sdy, sw, o, "e5m2", trans_b=False)
    m = orc.compare(pkg.as_bf16_bits(x.grad), ref_dx)
    _say(f"dgrad: {m}")
    assert orc.parity_ok(m)
    ref_dwt = orc.vark_wgrad_tensorwise(_bytes(qx), _bytes(qdy), sx, sdy, o)          # [G, K, N]
    m = orc.compare(pkg.as_bf16_bits(w.grad.transpose(1, 2)), ref_dwt, o)
    _say(f"wgrad: {m}")
    assert orc.parity_ok(m) and m["empty_zero"]

    # wiring against the unquantized layer (float64 on the CPU)
    xd, wd, dyd = x.detach().double().cpu(), w.detach().double().cpu(), dy.double().cpu()
    out64 = torch.zeros((M, N), dtype=torch.float64)
    dx64 = torch.zeros((M, K), dtype=torch.float64)
    dw64 = torch.zeros((G, N, K), dtype=torch.float64)
    for gi in range(G):
        lo, hi = int(o[gi]), int(o[gi + 1])
        out64[lo:hi] = xd[lo:hi] @ wd[gi].T
        dx64[lo:hi] = dyd[lo:hi] @ wd[gi]
        dw64[gi] = dyd[lo:hi].T @ xd[lo:hi]
    c = (_cos(out.cpu(), out64), _cos(x.grad.cpu(), dx64), _cos(w.grad.cpu(), dw64))
    _say(f"cosine to the unquantized layer (out, dx, dw): {c}")
    assert min(c) >= 0.99


def test_grouped_linear_fp8_main_grad(pkg, orc, cuda):
    """With main_grad the weight gradient is accumulated into the fp32 [G, K, N] buffer."""
    from ggemm_asm_amd.autograd import grouped_linear_fp8
    lens, K, N = [64, 0, 200], 192, 384
    g = torch.Generator().manual_seed(9)
    G, M = len(lens), sum(lens)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(cuda).requires_grad_(True)
    w = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16).to(cuda).requires_grad_(True)
    dy = (torch.randn((M, N), generator=g) * 1e-2).to(torch.bfloat16).to(cuda)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    c0 = torch.randn((G, K, N), generator=g).to(cuda)
    mg = c0.clone()
    _say("grouped linear fp8 main_grad")
    grouped_linear_fp8(x, w, offs, main_grad=mg).backward(dy)
    torch.cuda.synchronize()
    assert w.grad is None and x.grad is not None
    qx, sx, _ = pkg.quantize_fp8_tensorwise(x.detach(), "e4m3")
    qdy, sdy, _ = pkg.quantize_fp8_tensorwise(dy, "e5m2")
    f32 = pkg.grouped_gemm_fp8_tensorwise_variable_k(qx, qdy, sx, sdy, offs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(mg, c0 + f32)


def test_grouped_linear_fp8_dropped_tokens_are_zero(pkg, orc, orp, cuda):
    """Routing that drops tokens (offs[G] < M): the rows past offs[G] of out and of x.grad are exact
    zeros, also when the buffers torch hands out held other values before (the first call fills
    the caching allocator's blocks with a full-routing run)."""
    from ggemm_asm_amd.autograd import grouped_linear_fp8
    lens, K, N, M = [100, 0, 157], 256, 384, 400
    g = torch.Generator().manual_seed(17)
    G = len(lens)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(cuda).requires_grad_(True)
    w = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16).to(cuda).requires_grad_(True)
    dy = (torch.randn((M, N), generator=g) * 1e-2).to(torch.bfloat16).to(cuda)
    full = torch.tensor([0, 100, 100, M], dtype=torch.int64, device=cuda)
    _say("grouped linear fp8 with dropped tokens")
    grouped_linear_fp8(x, w, full).backward(dy)      # leaves nonzero values in freed blocks
    x.grad = None
    w.grad = None
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    out = grouped_linear_fp8(x, w, offs)
    out.backward(dy)
    torch.cuda.synchronize()
    end = int(sum(lens))
    assert bool((out[end:].view(torch.int16) == 0).all())
    assert bool((x.grad[end:].view(torch.int16) == 0).all())
    qx, sx, _ = pkg.quantize_fp8_tensorwise(x.detach(), "e4m3")
    qw, sw, _ = pkg.quantize_fp8_tensorwise(w.detach(), "e4m3")
    o = offs.cpu().numpy()
    ref_out = orp.grouped_fp8(_bytes(qx)[:end], _bytes(qw), float(sx), float(sw), o, "e4m3")
    m = orc.compare(pkg.as_bf16_bits(out)[:end], ref_out)
    _say(f"forward rows within offs[G]: {m}")
    assert orc.parity_ok(m)


def test_grouped_linear_fp8_weight_cache(pkg, cuda):
    """weight_cache: the second call with an unchanged weight reuses its fp8 copy and gives the
    same bits as an uncached call; an in-place update of the weight quantizes again; a call that
    needs the data gradient after one that did not upgrades the entry with q^T."""
    from ggemm_asm_amd.autograd import FP8WeightCache, grouped_linear_fp8
    lens, K, N = [96, 0, 160], 192, 256
    g = torch.Generator().manual_seed(23)
    G, M = len(lens), sum(lens)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(cuda)
    w = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16).to(cuda).requires_grad_(True)
    dy = (torch.randn((M, N), generator=g) * 1e-2).to(torch.bfloat16).to(cuda)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    cache = FP8WeightCache()
    _say("grouped linear fp8 weight cache")
    out0 = grouped_linear_fp8(x, w, offs, weight_cache=cache)      # x needs no grad: no q^T
    assert (cache.hits, cache.misses) == (0, 1)
    xg = x.clone().requires_grad_(True)
    out1 = grouped_linear_fp8(xg, w, offs, weight_cache=cache)     # needs q^T: upgraded
    assert (cache.hits, cache.misses) == (0, 2)
    out1.backward(dy)
    dx_ref = xg.grad.clone()
    xg.grad = None
    out2 = grouped_linear_fp8(xg, w, offs, weight_cache=cache)     # hit
    assert (cache.hits, cache.misses) == (1, 2)
    out2.backward(dy)
    ref = grouped_linear_fp8(x, w.detach(), offs)                  # uncached
    torch.cuda.synchronize()
    for o in (out0, out1, out2):
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(xg.grad.view(torch.int16), dx_ref.view(torch.int16))
    with torch.no_grad():
        w.mul_(2.0)                                                # an optimizer-like in-place step
    out3 = grouped_linear_fp8(x, w, offs, weight_cache=cache)
    assert (cache.hits, cache.misses) == (1, 3)
    ref3 = grouped_linear_fp8(x, w.detach(), offs)
    torch.cuda.synchronize()
    assert torch.equal(out3.view(torch.int16), ref3.view(torch.int16))
    assert not torch.equal(out3.view(torch.int16), ref.view(torch.int16))


def test_grouped_linear_fp8_delayed_scaling(pkg, orc, orp, cuda):
    """scaling=FP8DelayedScaling: with the same x, w and dy every step the histories hold their own
    amax, so every output and gradient equals the current-scaling op's bit for bit; a step whose
    x and dy shrink quantizes them with the scale of the history (the previous steps' larger
    amax), which the forward, dgrad and wgrad against the oracle on those bytes confirm, and
    records their amax in the slot. With a weight cache the weight role advances on misses only."""
    from ggemm_asm_amd.autograd import FP8DelayedScaling, grouped_linear_fp8
    lens, K, N = [96, 0, 160, 64], 192, 256
    g = torch.Generator().manual_seed(29)
    G, M = len(lens), sum(lens)
    x0 = torch.randn((M, K), generator=g).to(torch.bfloat16).to(cuda)
    w = (torch.randn((G, N, K), generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    dy = (torch.randn((M, N), generator=g) * 1e-2).to(torch.bfloat16).to(cuda)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    o = offs.cpu().numpy()

    def step(xv, dyv, scaling):
        xg, wg = xv.clone().requires_grad_(True), w.clone().requires_grad_(True)
        out = grouped_linear_fp8(xg, wg, offs, scaling=scaling)
        out.backward(dyv)
        return out, xg.grad, wg.grad

    rec = FP8DelayedScaling(history_len=4)
    _say("grouped linear fp8 delayed scaling: constant steps")
    ref = step(x0, dy, None)
    for n in range(3):
        got = step(x0, dy, rec)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), n
    assert rec.calls == {"x": 3, "w": 3, "dy": 3}
    hx, hdy = rec.history["x"].clone(), rec.history["dy"].clone()
    ax, ady, aw = float(pkg.amax(x0)), float(pkg.amax(dy)), float(pkg.amax(w))
    assert hx.tolist() == [ax, ax, ax, 0.0] and hdy.tolist() == [ady, ady, ady, 0.0]
    assert rec.history["w"].tolist() == [aw, aw, aw, 0.0]

    _say("grouped linear fp8 delayed scaling: shrinking step")
    x1, dy1 = (x0.float() * 0.5).to(torch.bfloat16), (dy.float() * 0.25).to(torch.bfloat16)
    out, dx, dw = step(x1, dy1, rec)
    torch.cuda.synchronize()
    assert rec.calls == {"x": 4, "w": 4, "dy": 4}
    assert float(rec.history["x"][3]) == float(pkg.amax(x1)) and float(rec.history["dy"][3]) == float(pkg.amax(dy1))
    qx, sx = pkg.quantize_fp8_tensorwise_delayed(x1, hx, 3, "e4m3")
    qdy, sdy = pkg.quantize_fp8_tensorwise_delayed(dy1, hdy, 3, "e5m2")
    qw, sw, _ = pkg.quantize_fp8_tensorwise(w, "e4m3")
    assert float(sx) == float(np.float32(ax) / np.float32(448.0))
    assert float(sdy) == float(np.float32(ady) / np.float32(57344.0))
    m = orc.compare(pkg.as_bf16_bits(out), orp.grouped_fp8(_bytes(qx), _bytes(qw), float(sx), float(sw), o, "e4m3"))
    _say(f"forward: {m}")
    assert orc.parity_ok(m)
    m = orc.compare(pkg.as_bf16_bits(dx), orp.grouped_fp8(_bytes(qdy), _bytes(qw), float(sdy), float(sw), o, "e5m2",
                                                          trans_b=False))
    _say(f"dgrad: {m}")
    assert orc.parity_ok(m)
    m = orc.compare(pkg.as_bf16_bits(dw.transpose(1, 2)),
                    orc.vark_wgrad_tensorwise(_bytes(qx), _bytes(qdy), float(sx), float(sdy), o), o)
    _say(f"wgrad: {m}")
    assert orc.parity_ok(m)
    ref64 = torch.cat([x1[o[i]:o[i + 1]].double() @ w[i].double().T for i in range(G)])
    assert _cos(out, ref64) >= 0.99

    _say("grouped linear fp8 delayed scaling with a weight cache")
    from ggemm_asm_amd.autograd import FP8WeightCache
    rec2, cache = FP8DelayedScaling(history_len=4), FP8WeightCache()
    wg = w.clone().requires_grad_(True)
    for n in range(3):
        xg = x0.clone().requires_grad_(True)
        out = grouped_linear_fp8(xg, wg, offs, weight_cache=cache, scaling=rec2)
        out.backward(dy)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref[0].view(torch.int16)), n
        assert torch.equal(xg.grad.view(torch.int16), ref[1].view(torch.int16)), n
    assert rec2.calls == {"x": 3, "w": 1, "dy": 3} and (cache.hits, cache.misses) == (2, 1)
