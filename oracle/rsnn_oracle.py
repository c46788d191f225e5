"""CPU oracle of the recurrent spiking-network trainer (atlas_rsnn_* in libatlas_train_hip.so).

TEST INFRASTRUCTURE ONLY: the checker of the GPU trainer; only tests/ and bench.py's CPU-baseline
leg may import it.

The model is the benchmark's configuration 4 in the SpyTorch discretisation.  The reference's
training plans have spike-count rate logits only (brian2-rust/src/training/multistate.rs:186-206,
brian2-rust/python/brian2_rust/training_metal.metal:77-83): the leaky readout and the
max-over-time loss have no reference counterpart.  What pins this restatement is therefore
independent mathematics, as in the reference's own check of its VJP
(brian2-rust/tests/test_native_training.py:18-55):

* the adjoint ``backward`` equals torch autograd of an independently written forward with a
  custom surrogate function (tests/test_rsnn.py);
* it equals central finite differences of the frozen-anchor linearisation, in which every hard
  spike becomes s0 + sigma(m0) (m - m0) around the recorded trajectory and the reset keeps the
  recorded spike (the reset is not differentiated);
* ``adam`` equals torch.optim.Adam on the same gradients.

Every quantity is float64 unless ``dtype`` says otherwise.
"""
from __future__ import annotations

import numpy as np


def forward(spec: dict, w_in, w_rec, w_out, x, labels, *, teacher=None, anchors=None, dtype=np.float64) -> dict:
    """Run the network over x[B, T, I].

    ``teacher`` (spikes [T, B, H]) replaces the network's own spikes everywhere they are used
    (recurrence, reset and readout), so each tick is checked against a device run without the
    chaotic divergence that a single flipped spike starts; it also returns ``mem_scale``, the
    membrane recurrence run over absolute values, the magnitude a float32 rounding error of each
    membrane is relative to, and ``logit_scale``, the same for the logits.  ``anchors`` = (mem_tape, spikes) applies the frozen-anchor
    linearisation.
    """
    f = lambda a: np.asarray(a, dtype)
    x, w_in, w_rec, w_out = f(x), f(w_in), f(w_rec), f(w_out)
    alpha, beta, theta, slope = (dtype(spec[k]) for k in ("alpha", "beta", "threshold", "slope"))
    B, T, _ = x.shape
    H, C = w_rec.shape[0], w_out.shape[1]
    syn = np.zeros((B, H), dtype)
    mem = np.zeros((B, H), dtype)
    previous = np.zeros((B, H), dtype)
    mem_tape = np.zeros((T, B, H), dtype)
    spikes = np.zeros((T, B, H), dtype)
    hin = x.transpose(1, 0, 2) @ w_in             # [T, B, H]
    for t in range(T):
        hard = (mem > theta).astype(dtype)
        if teacher is not None:
            hard = np.asarray(teacher[t], dtype)
        s, reset = hard, hard
        if anchors is not None:
            m0, s0 = anchors[0][t], anchors[1][t]
            s = s0 + _sigma(m0, theta, slope) * (mem - m0)
            reset = s0
        mem_tape[t] = mem
        spikes[t] = s
        h1 = hin[t] + previous @ w_rec
        syn, mem = alpha * syn + h1, (beta * mem + syn) * (1 - reset)
        previous = s
    if teacher is not None:
        # magnitude of the terms that produced each state: the same recurrence over absolute
        # values, the scale a float32 evaluation's rounding error is relative to
        mag = np.zeros((T, B, H), dtype)
        syn_a = np.zeros((B, H), dtype)
        mem_a = np.zeros((B, H), dtype)
        hin_a = np.abs(x.transpose(1, 0, 2)) @ np.abs(w_in)
        for t in range(T):
            mag[t] = mem_a
            h1_a = hin_a[t] + (np.abs(spikes[t - 1]) @ np.abs(w_rec) if t else 0.0)
            syn_a, mem_a = alpha * syn_a + h1_a, (beta * mem_a + syn_a) * (1 - np.asarray(teacher[t], dtype))
    h2 = spikes @ w_out
    f_state = np.zeros((B, C), dtype)
    u = np.zeros((B, C), dtype)
    trace = [u]
    for t in range(T):
        f_state, u = alpha * f_state + h2[t], beta * u + f_state
        trace.append(u)
    trace = np.stack(trace)                       # U_0 .. U_T, [T + 1, B, C]
    index = trace.argmax(axis=0)                  # first maximum
    logits = np.take_along_axis(trace, index[None], axis=0)[0]
    top = logits.max(axis=1)
    lse = top + np.log(np.exp(logits - top[:, None]).sum(axis=1))
    logit_scale = None
    if teacher is not None:
        # the readout recurrence over |s| |W_out| at the same tick: each logit's term magnitude
        f_a = np.zeros((B, C), dtype)
        u_a = np.zeros((B, C), dtype)
        h2_a = np.abs(spikes) @ np.abs(w_out)
        trace_a = [u_a]
        for t in range(T):
            f_a, u_a = alpha * f_a + h2_a[t], beta * u_a + f_a
            trace_a.append(u_a)
        logit_scale = np.take_along_axis(np.stack(trace_a), index[None], axis=0)[0]
    labels = np.asarray(labels, np.int64)
    losses = lse - logits[np.arange(B), labels]
    soft = np.exp(logits - lse[:, None])
    onehot = np.zeros_like(soft)
    onehot[np.arange(B), labels] = 1
    return {"mem_tape": mem_tape, "mem_scale": mag if teacher is not None else None, "spikes": spikes, "h2": h2,
            "trace": trace, "argmax": index - 1, "logit_scale": logit_scale,
            "logits": logits, "losses": losses, "loss": losses.mean(), "glogit": (soft - onehot) / B}


def _sigma(mem, theta, slope):
    return 1.0 / (slope * np.abs(mem - theta) + 1.0) ** 2


def backward(spec: dict, w_in, w_rec, w_out, x, fwd: dict) -> dict:
    """Adjoint of ``forward`` (its hard-spike trajectory, surrogate derivative, reset not
    differentiated): the gradients of the mean loss with respect to the three weights."""
    x = np.asarray(x, np.float64)
    w_rec = np.asarray(w_rec, np.float64)
    w_out = np.asarray(w_out, np.float64)
    alpha, beta, theta, slope = (float(spec[k]) for k in ("alpha", "beta", "threshold", "slope"))
    T, B, H = fwd["spikes"].shape
    C = w_out.shape[1]
    spikes = np.asarray(fwd["spikes"], np.float64)
    mem_tape = np.asarray(fwd["mem_tape"], np.float64)
    # readout: adjoint of F_{t+1} for every tick; the logit is U_{arg+1}
    gh2 = np.zeros((T, B, C))
    gu = np.zeros((B, C))
    gf = np.zeros((B, C))
    for t in reversed(range(T)):
        gu = gu + np.where(fwd["argmax"] == t, fwd["glogit"], 0.0)
        gh2[t] = gf
        gu, gf = beta * gu, gu + alpha * gf
    gs_read = gh2 @ w_out.T
    g1 = np.zeros((T, B, H))                      # adjoint of h1_t (= of syn_{t+1})
    gmem = np.zeros((B, H))
    gsyn = np.zeros((B, H))
    for t in reversed(range(T)):
        g1[t] = gsyn
        gs = gs_read[t] + (g1[t + 1] @ w_rec.T if t + 1 < T else 0.0)
        keep = 1 - spikes[t]
        gmem, gsyn = beta * keep * gmem + gs * _sigma(mem_tape[t], theta, slope), keep * gmem + alpha * gsyn
    rows = lambda a: a.reshape(-1, a.shape[-1])   # (tick, sample) rows
    return {"w_in": rows(x.transpose(1, 0, 2)).T @ rows(g1),
            "w_rec": rows(spikes[:-1]).T @ rows(g1[1:]),
            "w_out": rows(spikes).T @ rows(gh2)}


def adam(weights, moments, gradients, step: int, *, lr, beta1, beta2, epsilon):
    """One bias-corrected Adam update in float64; returns (weights, (m, v))."""
    m, v = moments
    m = beta1 * m + (1 - beta1) * gradients
    v = beta2 * v + (1 - beta2) * gradients ** 2
    update = lr * (m / (1 - beta1 ** step)) / (np.sqrt(v / (1 - beta2 ** step)) + epsilon)
    return weights - update, (m, v)
