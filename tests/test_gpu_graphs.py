"""HIP graph capture of the library's launches (torch.cuda.CUDAGraph over the C ABI).

One training step's kernels at a small shape -- the producer (per-tensor, with the transposed weight
copy, line-aligned rows), the persistent forward and data-gradient GEMMs, the variable-K wgrad in
bf16 and accumulating into an fp32 main-grad -- are captured once and replayed several times, with
eager work of the same library between replays (as a training loop would interleave it), and every
replay is compared with the eager results bit for bit, including a replay after the inputs were
overwritten in place (the graph reads its inputs, not copies). The launches record no memset: the
amax result is cleared by a fill kernel. A second test captures the autograd op's forward and
backward (torch.autograd.grad) in one graph; a third the delayed-scaling quantizers with a fixed
history slot.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def test_graph_replays_match_eager(pkg, cuda):
    lens, K, N = [300, 0, 517, 64], 256, 384
    G, M = len(lens), sum(lens)
    g = torch.Generator(device=cuda).manual_seed(0)

    def inputs():
        x = torch.randn((M, K), generator=g, device=cuda).to(torch.bfloat16)
        w = (torch.randn((G, N, K), generator=g, device=cuda) * 0.05).to(torch.bfloat16)
        dy = (torch.randn((M, N), generator=g, device=cuda) * 1e-2).to(torch.bfloat16)
        return x, w, dy

    x, w, dy = inputs()
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    main_grad = torch.zeros((G, K, N), dtype=torch.float32, device=cuda)

    def step():
        qx, sx, _ = pkg.quantize_fp8_tensorwise(x, "e4m3", row_align=128)
        qw, qwt, sw, _ = pkg.quantize_fp8_tensorwise_transpose(w, "e4m3", row_align=128)
        out = pkg.grouped_gemm_fp8_tensorwise(qx, qw, sx, sw, offs)
        qdy, sdy, _ = pkg.quantize_fp8_tensorwise(dy, "e5m2", row_align=128)
        dx = pkg.grouped_gemm_fp8_tensorwise(qdy, qwt, sdy, sw, offs)
        dw = pkg.grouped_gemm_fp8_tensorwise_variable_k(qx, qdy, sx, sdy, offs)
        pkg.grouped_gemm_fp8_tensorwise_variable_k(qx, qdy, sx, sdy, offs, out=main_grad, accumulate=True)
        return out, dx, dw

    _say("graph capture: eager reference")
    ref = [t.clone() for t in step()]
    dw32 = main_grad.clone()                     # one accumulation of the fp32 wgrad into zeros
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    _say("graph capture: capturing")
    with torch.cuda.graph(graph):
        static = step()
    torch.cuda.synchronize()

    for r in range(3):
        _say(f"graph replay {r}")
        pkg.quantize_fp8_tensorwise(dy, "e4m3")            # eager work of the library between replays
        for t in static:
            t.fill_(float("nan"))
        main_grad.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dx", "dw"), static, ref):
            assert torch.equal(_bits(a), _bits(b)), (r, name)
        assert torch.equal(main_grad, dw32), r

    _say("graph replay with new inputs")
    x2, w2, dy2 = inputs()
    x.copy_(x2)
    w.copy_(w2)
    dy.copy_(dy2)
    main_grad.zero_()
    want = [t.clone() for t in step()]
    want32 = main_grad.clone()
    main_grad.zero_()
    graph.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(("out", "dx", "dw"), static, want):
        assert torch.equal(_bits(a), _bits(b)), name
    assert torch.equal(main_grad, want32)
    assert not torch.equal(_bits(want[2]), _bits(ref[2]))   # the inputs did change the result


def test_graph_captures_autograd_layer(pkg, cuda):
    """The autograd op's forward and backward (torch.autograd.grad) captured in one graph: replays
    equal eager out, dx and dw bit for bit, also after the inputs are overwritten in place."""
    from ggemm_asm_amd.autograd import grouped_linear_fp8
    lens, K, N = [257, 0, 96, 400], 192, 320
    G, M = len(lens), sum(lens)
    g = torch.Generator(device=cuda).manual_seed(1)
    x = torch.randn((M, K), generator=g, device=cuda).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn((G, N, K), generator=g, device=cuda) * 0.05).to(torch.bfloat16).requires_grad_(True)
    dy = (torch.randn((M, N), generator=g, device=cuda) * 1e-2).to(torch.bfloat16)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)

    def step():
        out = grouped_linear_fp8(x, w, offs)
        dx, dw = torch.autograd.grad(out, (x, w), dy)
        return out.detach(), dx, dw

    _say("graph autograd: eager")
    ref = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    _say("graph autograd: capturing")
    with torch.cuda.graph(graph):
        static = step()
    for r in range(2):
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dx", "dw"), static, ref):
            assert torch.equal(_bits(a), _bits(b)), (r, name)
    _say("graph autograd: new inputs")
    with torch.no_grad():
        x.mul_(-0.5)
        w.add_(0.01)
        dy.mul_(2.0)
    want = [t.clone() for t in step()]
    graph.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(("out", "dx", "dw"), static, want):
        assert torch.equal(_bits(a), _bits(b)), name


def test_graph_replays_delayed_quantizers(pkg, cuda):
    """The delayed-scaling quantizers (plain and transposing) captured with a fixed history slot:
    every replay, with eager calls of the same kernels on other data between replays, equals the
    eager bytes, scale and history; the graph reads the history at replay time (an entry changed in
    place changes the scale) and records this x's amax in the slot (x overwritten in place)."""
    g = torch.Generator(device=cuda).manual_seed(3)
    x = torch.randn((640, 384), generator=g, device=cuda).to(torch.bfloat16)
    w = (torch.randn((3, 160, 96), generator=g, device=cuda) * 0.05).to(torch.bfloat16)
    hx = torch.tensor([2.5, 0.0, 3.0, 1.0], device=cuda)
    hw = torch.tensor([0.1, 0.2, 0.0], device=cuda)
    other = torch.randn((256, 128), generator=g, device=cuda).to(torch.bfloat16)
    ho = torch.tensor([1.0, 0.0], device=cuda)

    def run():
        q, s = pkg.quantize_fp8_tensorwise_delayed(x, hx, 1, "e4m3", row_align=128)
        qw, qwt, sw = pkg.quantize_fp8_tensorwise_transpose_delayed(w, hw, 2, "e4m3", row_align=128)
        return q, s, qw, qwt, sw

    def snapshot(outs):
        return [t.view(torch.uint8).clone() if t.dtype.is_floating_point and t.element_size() == 1 else t.clone()
                for t in outs] + [hx.clone(), hw.clone()]

    def check(static, ref, tag):
        got = [t.view(torch.uint8) if t.element_size() == 1 else t for t in static] + [hx, hw]
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), (tag, i)

    _say("graph delayed quantizers: eager")
    ref = snapshot(run())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    _say("graph delayed quantizers: capturing")
    with torch.cuda.graph(graph):
        static = run()
    for r in range(3):
        pkg.quantize_fp8_tensorwise_delayed(other, ho, 1, "e5m2")       # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        check(static, ref, f"replay {r}")
    _say("graph delayed quantizers: history and input changed in place")
    with torch.no_grad():
        hx[0] = 40.0
        hw[1] = 0.05
        x.mul_(3.0)
    want = snapshot(run())
    with torch.no_grad():
        hx[1] = 0.0
        hw[2] = 0.0
    graph.replay()
    torch.cuda.synchronize()
    check(static, want, "changed")
    assert float(static[1]) == float(np.float32(40.0) / np.float32(448.0))
    assert float(hx[1]) == float(x.float().abs().max())
