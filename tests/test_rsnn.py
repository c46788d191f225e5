"""Pins of the recurrent-trainer oracle (oracle/rsnn_oracle.py) and the host side of the
configuration-4 plan.  The reference has no leaky-readout / max-over-time plan, so the oracle is
pinned by independent mathematics: torch autograd of a separately written forward, central
finite differences of the frozen-anchor linearisation (the method of
brian2-rust/tests/test_native_training.py:18-55) and torch.optim.Adam."""
import math

import numpy as np
import pytest
import torch

from atlas_hip import rsnn
from oracle import rsnn_oracle as ro

SPEC = {"alpha": math.exp(-1 / 5), "beta": math.exp(-1 / 20), "threshold": 1.0, "slope": 25.0}


def case(seed=0, B=4, T=24, I=12, H=16, C=5, scale=3.0, rate=0.15):
    rng = np.random.default_rng(seed)
    x = (rng.random((B, T, I)) < rate).astype(np.float64)
    labels = rng.integers(0, C, size=B)
    w = [rng.standard_normal(s) * scale / math.sqrt(s[0]) for s in ((I, H), (H, H), (H, C))]
    return x, labels, w


class _Spike(torch.autograd.Function):
    """Heaviside forward, fast-sigmoid derivative 1/(slope |v| + 1)^2 backward."""

    @staticmethod
    def forward(ctx, v, slope):
        ctx.save_for_backward(v)
        ctx.slope = slope
        return (v > 0).to(v.dtype)

    @staticmethod
    def backward(ctx, grad):
        (v,) = ctx.saved_tensors
        return grad / (ctx.slope * v.abs() + 1.0) ** 2, None


def torch_loss(spec, w_in, w_rec, w_out, x, labels):
    """SpyTorch-style network written independently of the oracle (per-tick loop, torch ops)."""
    B, T, _ = x.shape
    H, C = w_rec.shape[0], w_out.shape[1]
    syn = torch.zeros(B, H, dtype=x.dtype)
    mem = torch.zeros(B, H, dtype=x.dtype)
    out = torch.zeros(B, H, dtype=x.dtype)
    hin = torch.einsum("bti,ih->bth", x, w_in)
    recorded = []
    for t in range(T):
        out_t = _Spike.apply(mem - spec["threshold"], spec["slope"])
        rst = out_t.detach()
        h1 = hin[:, t] + out @ w_rec
        syn, mem = spec["alpha"] * syn + h1, (spec["beta"] * mem + syn) * (1.0 - rst)
        recorded.append(out_t)
        out = out_t
    spk = torch.stack(recorded, dim=1)
    h2 = torch.einsum("bth,hc->btc", spk, w_out)
    flt = torch.zeros(B, C, dtype=x.dtype)
    u = torch.zeros(B, C, dtype=x.dtype)
    trace = [u]
    for t in range(T):
        flt, u = spec["alpha"] * flt + h2[:, t], spec["beta"] * u + flt
        trace.append(u)
    logits, _ = torch.max(torch.stack(trace, dim=1), dim=1)
    return torch.nn.functional.cross_entropy(logits, labels), spk, logits


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_backward_matches_torch_autograd(seed):
    x, labels, w = case(seed)
    tw = [torch.tensor(a, requires_grad=True) for a in w]
    loss, spk, logits = torch_loss(SPEC, *tw, torch.tensor(x), torch.tensor(labels))
    loss.backward()
    fwd = ro.forward(SPEC, *w, x, labels)
    assert spk.sum() > 10, "case too quiet to exercise the surrogate"
    assert np.array_equal(fwd["spikes"], spk.detach().numpy().transpose(1, 0, 2))
    assert abs(fwd["loss"] - loss.item()) < 1e-12
    np.testing.assert_allclose(fwd["logits"], logits.detach().numpy(), rtol=0, atol=1e-12)
    grads = ro.backward(SPEC, *w, x, fwd)
    for key, t in zip(("w_in", "w_rec", "w_out"), tw):
        np.testing.assert_allclose(grads[key], t.grad.numpy(), rtol=1e-10, atol=1e-13, err_msg=key)
        assert np.abs(grads[key]).max() > 0, key


def test_backward_matches_frozen_anchor_finite_differences():
    x, labels, w = case(5, B=3, T=16, I=6, H=16, C=4)
    fwd = ro.forward(SPEC, *w, x, labels)
    anchors = (fwd["mem_tape"], fwd["spikes"])
    assert fwd["spikes"].sum() > 5
    # the anchored forward reproduces the hard trajectory at the anchor
    again = ro.forward(SPEC, *w, x, labels, anchors=anchors)
    assert abs(again["loss"] - fwd["loss"]) < 1e-14
    grads = ro.backward(SPEC, *w, x, fwd)
    rng = np.random.default_rng(7)
    eps = 1e-6
    for k, key in enumerate(("w_in", "w_rec", "w_out")):
        for flat in rng.choice(w[k].size, size=12, replace=False):
            idx = np.unravel_index(flat, w[k].shape)
            plus = [a.copy() for a in w]
            minus = [a.copy() for a in w]
            plus[k][idx] += eps
            minus[k][idx] -= eps
            fd = (ro.forward(SPEC, *plus, x, labels, anchors=anchors)["loss"] -
                  ro.forward(SPEC, *minus, x, labels, anchors=anchors)["loss"]) / (2 * eps)
            assert abs(fd - grads[key][idx]) <= 1e-7 + 1e-6 * abs(fd), (key, idx, fd, grads[key][idx])


def test_planted_mistake_is_caught_by_the_pins(monkeypatch):
    """A plausible slip in the oracle (the surrogate's square dropped) must fail the
    torch-autograd comparison."""
    x, labels, w = case(1)
    tw = [torch.tensor(a, requires_grad=True) for a in w]
    loss, _, _ = torch_loss(SPEC, *tw, torch.tensor(x), torch.tensor(labels))
    loss.backward()
    monkeypatch.setattr(ro, "_sigma", lambda mem, theta, slope: 1.0 / (slope * np.abs(mem - theta) + 1.0))
    fwd = ro.forward(SPEC, *w, x, labels)
    bad = ro.backward(SPEC, *w, x, fwd)
    assert not np.allclose(bad["w_in"], tw[0].grad.numpy(), rtol=1e-6, atol=1e-9)


def test_adam_matches_torch():
    rng = np.random.default_rng(3)
    w0 = rng.standard_normal((7, 5))
    p = torch.tensor(w0.copy(), requires_grad=True)
    opt = torch.optim.Adam([p], lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    w, mom = w0.copy(), (np.zeros_like(w0), np.zeros_like(w0))
    for step in range(1, 6):
        g = rng.standard_normal(w0.shape)
        p.grad = torch.tensor(g)
        opt.step()
        w, mom = ro.adam(w, mom, g, step, lr=1e-3, beta1=0.9, beta2=0.999, epsilon=1e-8)
    np.testing.assert_allclose(w, p.detach().numpy(), rtol=0, atol=1e-15)


def test_teacher_forcing_reproduces_the_free_run():
    x, labels, w = case(2)
    free = ro.forward(SPEC, *w, x, labels)
    forced = ro.forward(SPEC, *w, x, labels, teacher=free["spikes"])
    for key in ("mem_tape", "spikes", "logits", "losses"):
        assert np.array_equal(free[key], forced[key]), key


def test_poisson_batch_statistics():
    rng = np.random.default_rng(0)
    x, labels = rsnn.poisson_inputs(rng, 64, 100, 700, 20)
    assert x.shape == (64, 100, 700) and x.dtype == np.float32
    assert set(np.unique(x)) <= {0.0, 1.0}
    mean_rate = x.mean() / 1e-3
    assert 8.0 < mean_rate < 12.0            # E[rate] = 10 Hz
    assert labels.max() < 20


def test_plan_defaults_and_validation():
    plan = rsnn.recurrent_plan()
    assert plan["alpha"] == pytest.approx(math.exp(-1 / 5)) and plan["beta"] == pytest.approx(math.exp(-1 / 20))
    assert (plan["batch"], plan["time"], plan["inputs"], plan["hidden"], plan["classes"]) == (256, 100, 700, 256, 20)
    with pytest.raises(ValueError):
        rsnn.recurrent_plan(hidden=20)
    with pytest.raises(ValueError):
        rsnn.recurrent_plan(bogus=1)
    w = rsnn.initial_weights(plan, seed=1)
    assert [a.shape for a in w] == [(700, 256), (256, 256), (256, 20)]
    assert abs(float(w[0].std()) * math.sqrt(700) - 1) < 0.02
