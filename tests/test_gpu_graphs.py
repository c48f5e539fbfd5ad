"""HIP graph capture of the library's launches (torch.cuda.CUDAGraph over the C ABI).

One training step's kernels at a small shape -- the producer (per-tensor, with the transposed weight
copy, line-aligned rows), the persistent forward and data-gradient GEMMs, the variable-K wgrad in
bf16 and accumulating into an fp32 main-grad -- are captured once and replayed several times, with
eager work of the same library between replays (as a training loop would interleave it), and every
replay is compared with the eager results bit for bit, including a replay after the inputs were
overwritten in place (the graph reads its inputs, not copies). The launches record no memset: the
amax result is cleared by a fill kernel. A second test captures the autograd op's forward and
backward (torch.autograd.grad) in one graph; a third the delayed-scaling quantizers with a fixed
history slot; the last two the delayed-scaling quantizers and the autograd layer with device slots,
whose replays advance through the history.
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


def test_graph_replays_roll_device_slot(pkg, cuda):
    """The delayed-scaling quantizers with device slots captured once: every replay advances the
    slots and records into the next history entry, so replay n equals the eager host-slot call n
    (slot n % H) -- bytes, scales and histories -- with the inputs changed in place between replays
    and eager library work in between. A host slot would record into one entry on every replay."""
    g = torch.Generator(device=cuda).manual_seed(5)
    Hx, Hw = 4, 3
    mags = (1.0, 2.0, 0.5, 6.0, 1.0, 0.25, 3.0, 10.0)
    xs = [(torch.randn((640, 384), generator=g, device=cuda) * m).to(torch.bfloat16) for m in mags]
    ws = [(torch.randn((3, 160, 96), generator=g, device=cuda) * 0.05 * m).to(torch.bfloat16) for m in mags]
    x, w = xs[1].clone(), ws[1].clone()                          # call 0 (the seed) ran before
    hx = torch.tensor([float(xs[0].float().abs().max()), 0, 0, 0], device=cuda)   # seeded by call 0
    hw = torch.tensor([float(ws[0].float().abs().max()), 0, 0], device=cuda)
    sx = torch.zeros(1, dtype=torch.int32, device=cuda)          # the previous call's slot: 0
    sw = torch.zeros(1, dtype=torch.int32, device=cuda)
    hx_ref, hw_ref = hx.clone(), hw.clone()
    other = torch.randn((256, 128), generator=g, device=cuda).to(torch.bfloat16)
    ho = torch.tensor([1.0, 0.0], device=cuda)
    so = torch.zeros(1, dtype=torch.int32, device=cuda)

    def run():
        q, s = pkg.quantize_fp8_tensorwise_delayed(x, hx, sx, "e4m3", row_align=128)
        qw, qwt, s_w = pkg.quantize_fp8_tensorwise_transpose_delayed(w, hw, sw, "e4m3", row_align=128)
        return q, s, qw, qwt, s_w

    def reference(n):
        q, s = pkg.quantize_fp8_tensorwise_delayed(xs[n], hx_ref, n % Hx, "e4m3", row_align=128)
        qw, qwt, s_w = pkg.quantize_fp8_tensorwise_transpose_delayed(ws[n], hw_ref, n % Hw, "e4m3", row_align=128)
        return q, s, qw, qwt, s_w

    def check(got, want, n):
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, want)):
            a, b = (a.view(torch.uint8), b.view(torch.uint8)) if a.element_size() == 1 else (a, b)
            assert torch.equal(a, b), (n, i)
        assert torch.equal(hx, hx_ref) and torch.equal(hw, hw_ref), n
        assert int(sx) == n % Hx and int(sw) == n % Hw, n

    _say("graph device slots: eager call 1")
    check(run(), reference(1), 1)
    x.copy_(xs[2])
    w.copy_(ws[2])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        warm = run()                                              # call 2, the warm-up
    torch.cuda.current_stream().wait_stream(side)
    check(warm, reference(2), 2)
    graph = torch.cuda.CUDAGraph()
    _say("graph device slots: capturing")
    with torch.cuda.graph(graph):
        static = run()
    torch.cuda.synchronize()
    assert int(sx) == 2 and torch.equal(hx, hx_ref)               # capturing ran nothing
    for n in range(3, len(xs)):
        _say(f"graph device slots: replay for call {n}")
        x.copy_(xs[n])
        w.copy_(ws[n])
        pkg.quantize_fp8_tensorwise_delayed(other, ho, so, "e5m2")   # eager work between replays
        graph.replay()
        check(static, reference(n), n)


def test_graph_captures_autograd_layer_delayed_scaling(pkg, cuda):
    """The autograd layer with delayed scaling (FP8DelayedScaling, history 3) captured in one graph
    after two eager steps: each replay equals the step of an eager twin layer with its own recipe
    fed the same inputs -- out, dx and dw bit for bit -- while the input ranges change between
    replays, so a frozen history (a slot that did not advance) would change the scales."""
    from ggemm_asm_amd.autograd import FP8DelayedScaling, grouped_linear_fp8
    lens, K, N = [257, 0, 96, 400], 192, 320
    G, M = len(lens), sum(lens)
    g = torch.Generator(device=cuda).manual_seed(8)
    x0 = torch.randn((M, K), generator=g, device=cuda).to(torch.bfloat16)
    w0 = (torch.randn((G, N, K), generator=g, device=cuda) * 0.05).to(torch.bfloat16)
    dy0 = (torch.randn((M, N), generator=g, device=cuda) * 1e-2).to(torch.bfloat16)
    x = x0.clone().requires_grad_(True)
    w = w0.clone().requires_grad_(True)
    dy = dy0.clone()
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=cuda)
    rec_graph, rec_eager = FP8DelayedScaling(3), FP8DelayedScaling(3)
    factors = [(1.0, 1.0, 1.0), (2.0, 0.5, 3.0), (0.25, 1.0, 0.5), (4.0, 2.0, 8.0), (1.0, 0.25, 1.0),
               (0.5, 3.0, 0.125), (8.0, 1.0, 2.0)]

    def set_inputs(n):
        fx, fw, fd = factors[n]
        with torch.no_grad():
            x.copy_(x0 * fx)
            w.copy_(w0 * fw)
            dy.copy_(dy0 * fd)

    def step(rec):
        out = grouped_linear_fp8(x, w, offs, scaling=rec)
        dx, dw = torch.autograd.grad(out, (x, w), dy)
        return out.detach(), dx, dw

    def check(got, n):
        want = step(rec_eager)
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dx", "dw"), got, want):
            assert torch.equal(_bits(a), _bits(b)), (n, name)

    _say("graph autograd delayed: eager steps 0 and 1")
    set_inputs(0)
    check([t.clone() for t in step(rec_graph)], 0)
    set_inputs(1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        warm = [t.clone() for t in step(rec_graph)]
    torch.cuda.current_stream().wait_stream(side)
    check(warm, 1)
    graph = torch.cuda.CUDAGraph()
    _say("graph autograd delayed: capturing")
    with torch.cuda.graph(graph):
        static = step(rec_graph)
    for n in range(2, len(factors)):
        _say(f"graph autograd delayed: replay for step {n}")
        set_inputs(n)
        graph.replay()
        check(static, n)
    # the scales did move with the inputs: the last replay differs from current scaling's result
    out_cur = grouped_linear_fp8(x.detach(), w.detach(), offs)
    assert not torch.equal(_bits(static[0]), _bits(out_cur))
