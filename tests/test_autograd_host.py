"""CPU checks of the autograd layer's host-side state: the FP8 weight cache's hit/miss rules and the
delayed-scaling recipe's refusal to seed a history inside a graph capture. The quantization itself
is replaced by a stub that counts calls (these are rules about when to quantize, not numerics; the
GPU tests cover the numerics)."""
import pytest
import torch

from __graft_entry__ import load_package

load_package()
from ggemm_asm_amd import autograd  # noqa: E402


@pytest.fixture
def stub(monkeypatch):
    calls = []

    def fake_quantize_weight(w, with_transpose, scaling=None):
        calls.append(with_transpose)
        return ("qw", "qwt" if with_transpose else None, "scale")

    monkeypatch.setattr(autograd, "_quantize_weight", fake_quantize_weight)
    return calls


def test_cache_hits_until_an_in_place_write(stub):
    w = torch.randn(2, 16, 8)
    cache = autograd.FP8WeightCache()
    cache.get(w, True)
    cache.get(w, True)
    cache.get(w, False)        # an entry with q^T serves a call without the data gradient
    assert (cache.hits, cache.misses) == (2, 1)
    with torch.no_grad():
        w.add_(1.0)            # bumps w's version counter
    cache.get(w, True)
    assert (cache.hits, cache.misses) == (2, 2)


def test_cache_upgrades_an_entry_without_transpose(stub):
    w = torch.randn(2, 16, 8)
    cache = autograd.FP8WeightCache()
    cache.get(w, False)
    cache.get(w, True)
    assert stub == [False, True] and cache.misses == 2


def test_data_writes_are_not_seen_without_invalidate(stub):
    """A write through ``w.data`` (a tensor with its own version counter) does not change the
    cache key: documented as not detected. ``invalidate()`` makes the next call quantize."""
    w = torch.randn(2, 16, 8)
    cache = autograd.FP8WeightCache()
    cache.get(w, True)
    v = w._version
    w.data.mul_(2.0)
    assert w._version == v
    cache.get(w, True)
    assert (cache.hits, cache.misses) == (1, 1)      # stale entry served: the documented limit
    cache.invalidate()
    cache.get(w, True)
    assert (cache.hits, cache.misses) == (1, 2)


def test_attach_invalidates_after_optimizer_step(stub):
    """``attach(optimizer)`` drops the entry after every step, also when the optimizer writes the
    weight where the version counter does not see it (here: through ``.data`` in a custom step)."""
    w = torch.nn.Parameter(torch.randn(2, 16, 8))

    class RawSGD(torch.optim.Optimizer):
        def __init__(self, params):
            super().__init__(params, {"lr": 0.1})

        @torch.no_grad()
        def step(self, closure=None):
            for group in self.param_groups:
                for p in group["params"]:
                    p.data.add_(p.grad.data, alpha=-group["lr"])   # invisible to p._version

    opt = RawSGD([w])
    cache = autograd.FP8WeightCache()
    handle = cache.attach(opt)
    cache.get(w, True)
    w.grad = torch.ones_like(w)
    opt.step()
    cache.get(w, True)
    assert (cache.hits, cache.misses) == (0, 2)
    cache.get(w, True)
    assert (cache.hits, cache.misses) == (1, 2)
    handle.remove()
    opt.step()
    cache.get(w, True)
    assert (cache.hits, cache.misses) == (2, 2)      # detached: the raw write goes unseen again


def test_cache_misses_for_a_new_tensor_at_the_same_address(stub):
    w = torch.randn(2, 16, 8)
    cache = autograd.FP8WeightCache()
    cache.get(w, True)
    w2 = w.view(2, 16, 8)      # same storage, another tensor object
    cache.get(w2, True)
    assert cache.misses == 2


def test_delayed_scaling_refuses_to_seed_inside_a_capture(monkeypatch):
    """The first call of a role quantizes with current scaling and seeds the history: inside a
    graph capture that would freeze current scaling into every replay, so it raises instead."""
    rec = autograd.FP8DelayedScaling(4)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="must run eagerly"):
        rec.quantize("x", torch.zeros(16, 64), "e4m3")
    with pytest.raises(RuntimeError, match="must run eagerly"):
        rec.quantize_weight(torch.zeros(2, 16, 64), True)
    assert rec.history == {} and rec.calls == {}
