"""Independent float64 NumPy forward of the dense LIF training plan and its frozen-anchor
surrogate linearisation (the method of test_native_training.py:18-55), for finite-difference
checks of the declared VJP."""
import numpy as np


def forward(plan, weights, inputs, labels, initial=None, anchors=None):
    """(mean loss, spikes [B,T,N], final state [B,N], (membranes, spikes)).  With ``anchors``
    the hard spikes become s = s0 + phi(u0) (u - u0) around the recorded baseline, and the reset
    uses the recorded spike when the reset is detached."""
    inputs = np.asarray(inputs, np.float64)
    batch, time, _ = inputs.shape
    sizes = plan["sizes"]
    offsets = np.cumsum([0, *sizes[1:]])
    n = offsets[-1]
    state = np.zeros((batch, n)) if initial is None else np.asarray(initial, np.float64).copy()
    threshold = np.repeat(plan["threshold"], sizes[1:])
    beta = np.repeat(plan["beta"], sizes[1:])
    spikes, membranes = [], []
    for t in range(time):
        u = beta * state
        hard = (u > threshold).astype(float)
        s, reset_spike = hard.copy(), hard.copy()
        if anchors is not None:
            base_u, base_s = anchors
            phi = plan["surrogate"]["scale"] / (1 + plan["surrogate"]["slope"] * np.abs(base_u[:, t] - threshold)) ** 2
            s = base_s[:, t] + phi * (u - base_u[:, t])
            reset_spike = base_s[:, t] if plan["detach_reset"] else s
        state = u.copy()
        for l in range(len(sizes) - 1):
            x = inputs[:, t] if l == 0 else s[:, offsets[l - 1]:offsets[l]]
            w = np.asarray(weights[l], np.float64).reshape(sizes[l], sizes[l + 1])
            state[:, offsets[l]:offsets[l + 1]] += x @ w
        if plan["reset"] == "zero":
            state *= 1 - reset_spike
        else:
            state -= threshold * reset_spike
        spikes.append(s.copy())
        membranes.append(u.copy())
    spikes = np.stack(spikes, axis=1)
    membranes = np.stack(membranes, axis=1)
    logits = spikes[:, :, offsets[-2]:].mean(axis=1) * plan["logit_scale"]
    top = logits.max(axis=1)
    loss = np.mean(top + np.log(np.exp(logits - top[:, None]).sum(axis=1)) - logits[np.arange(batch), labels])
    return loss, spikes, state, (membranes, spikes)


def fd_weight_gradients(plan, weights, inputs, labels, initial, epsilon=1e-6):
    _, _, _, anchors = forward(plan, weights, inputs, labels, initial)
    out = []
    for l, row in enumerate(weights):
        grads = []
        for e in range(len(row)):
            plus = [list(r) for r in weights]
            minus = [list(r) for r in weights]
            plus[l][e] += epsilon
            minus[l][e] -= epsilon
            grads.append((forward(plan, plus, inputs, labels, initial, anchors)[0] -
                          forward(plan, minus, inputs, labels, initial, anchors)[0]) / (2 * epsilon))
        out.append(np.array(grads))
    return out


def graph_forward(plan, weights, inputs, labels, initial, anchors=None):
    """Independent float64 forward of a projection-graph plan (the method of
    test_native_training_graph.py:38-74): tied parameters expanded into one dense matrix per
    projection with np.add.at (masks applied), every layer's threshold before any projection,
    then the reset.  With ``anchors`` (u, s, starts of a baseline run) the spikes are linearised
    around the baseline and each TBPTT boundary restarts from the baseline's membrane.
    Returns (mean loss, spikes, final state, logits, anchors)."""
    x = np.asarray(inputs, np.float64)
    batch, time, _ = x.shape
    sizes = plan["sizes"]
    offsets = np.cumsum([0, *sizes[1:]])
    v = np.asarray(initial, np.float64).copy()
    thresholds = np.repeat(plan["threshold"], sizes[1:])
    beta = np.repeat(plan["beta"], sizes[1:])
    matrices = []
    for q, (p, w) in enumerate(zip(plan["projections"], weights)):
        matrix = np.zeros((sizes[p["source_layer"]], sizes[p["target_layer"]]))
        values = np.asarray(w, np.float64)[p["parameter_ids"]] * np.asarray(plan["masks"][q])[p["parameter_ids"]]
        np.add.at(matrix, (p["sources"], p["targets"]), values)
        matrices.append(matrix)
    spikes, pres, starts = [], [], []
    window = plan["tbptt_window"]
    for t in range(time):
        if anchors is not None and window and t > 0 and t % window == 0:
            v = anchors[2][:, t].copy()
        starts.append(v.copy())
        u = beta * v
        hard = (u > thresholds).astype(float)
        spike, reset_spike = hard, hard
        if anchors is not None:
            base_u, base_s, _ = anchors
            phi = plan["surrogate"]["scale"] / (1 + plan["surrogate"]["slope"] * abs(base_u[:, t] - thresholds)) ** 2
            spike = base_s[:, t] + phi * (u - base_u[:, t])
            reset_spike = base_s[:, t] if plan["detach_reset"] else spike
        v = u.copy()
        for p, matrix in zip(plan["projections"], matrices):
            source, target = p["source_layer"], p["target_layer"]
            row = x[:, t] if source == 0 else spike[:, offsets[source - 1]:offsets[source]]
            v[:, offsets[target - 1]:offsets[target]] += row @ matrix
        v = v * (1 - reset_spike) if plan["reset"] == "zero" else v - thresholds * reset_spike
        pres.append(u.copy())
        spikes.append(spike.copy())
    spikes = np.stack(spikes, axis=1)
    logits = spikes[:, :, offsets[-2]:].mean(axis=1) * plan["logit_scale"]
    top = logits.max(axis=1)
    loss = np.mean(top + np.log(np.exp(logits - top[:, None]).sum(axis=1)) - logits[np.arange(batch), labels])
    return loss, spikes, v, logits, (np.stack(pres, axis=1), spikes, np.stack(starts, axis=1))
