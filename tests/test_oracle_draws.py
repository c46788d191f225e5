"""Draw-by-draw pins of the oracle's binomial and Poisson samplers (counter_binomial,
counter_poisson: executor.rs:224-323), which PoissonInput and poisson() use.

Each draw is recomputed from the counter uniforms (counter_uniform_draw, whose mix64 the
published splitmix64 sequences pin in test_oracle.py) by the sampler's mathematical
definition in 60-digit arithmetic (mpmath), not by the oracle's floating-point recurrences:

* inversion (binomial, and its reversed tail for p > 1/2): the smallest k with
  u <= CDF(k), the CDF summed from C(n, k) p^k q^(n-k) with the exact q = 1 - p; a search
  that passes the restart bound min(n, n p + 10 sqrt(n p q + 1)) takes the next draw;
* the normal approximation (n p > 5 and n (1 - p) > 5): counter_normal sqrt(n p (1 - p)) + n p;
* the product method (poisson, lambda < 10): the smallest k with sum_{i<=k} ln u_i <= -lambda;
* PTRS (poisson, lambda >= 10; Hoermann, "The transformed rejection method for generating
  Poisson random variables", Insurance: Mathematics and Economics 12 (1993) 39-45): each
  trial's candidate floor((2a/us + b) u + lambda + 0.43), its squeeze and its acceptance test
  ln(v alpha^-1 / (a/us^2 + b)) <= -lambda + k ln lambda - ln k!, with the exact ln Gamma
  in place of the reference's Lanczos series.

The oracle must agree exactly, in both its libm and shared-math modes, except at ties: a
decision whose exact margin is below the floating-point error of the oracle's evaluation
(1e-9 absolute for quantities of order one, 1e-12 of the terms' magnitude for PTRS at large
lambda; fewer than one in a thousand of these cases).  Ties are counted, and each tie's
oracle value must be one of the two the decision allows.
"""
import math

import mpmath
import numpy as np
import pytest

from oracle import oracle

mp = mpmath.mp
mp.dps = 60
MASK = (1 << 64) - 1
TIE = mpmath.mpf("1e-9")
RELATIVE = mpmath.mpf("1e-12")


def mix64(v: int) -> int:
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & MASK
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & MASK
    return v ^ (v >> 31)


def uniform(seed: int, stream: int, tick: int, index: int, draw: int) -> float:
    """counter_uniform_draw (executor.rs:196-203): 53 bits of mix64 of the counter."""
    c = (seed ^ (stream * 0x9E3779B97F4A7C15) ^ (tick * 0xD1B54A32D192ED03) ^ (index * 0x94D049BB133111EB)
         ^ (draw * 0x369DEA0F31A53F85)) & MASK
    return (mix64(c) >> 11) * 2.0 ** -53


def keys(count: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(count):
        yield (int(rng.integers(0, 2 ** 63)), int(rng.integers(0, 10 ** 6)), int(rng.integers(0, 10 ** 6)),
               int(rng.integers(0, 10 ** 6)))


# ------------------------------------------------------------------ binomial
def inversion(u: float, n: int, pr: float):
    """The smallest k with u <= CDF(k) of Binomial(n, pr), pr <= 1/2, or -1 once k passes the
    restart bound; and whether the decision is a tie."""
    P = mpmath.mpf(pr)
    Q = 1 - P
    bound = min(mpmath.mpf(n), n * P + 10 * mpmath.sqrt(n * P * Q + 1))
    U = mpmath.mpf(u)
    below = mpmath.mpf(0)
    k = 0
    while True:
        cdf = below + mpmath.binomial(n, k) * P ** k * Q ** (n - k)
        if U <= cdf:
            tie = (cdf - U) < TIE or (k > 0 and U - below < TIE)
            return k, tie
        k += 1
        if k > bound:
            return -1, abs(bound - mpmath.nint(bound)) < TIE
        below = cdf


def exact_binomial(key, n: int, p: float, approximate: bool):
    """The draw of counter_binomial by definition; (value, ties, restarts)."""
    if p <= 0:
        return 0.0, 0, 0
    if p >= 1:
        return float(n), 0, 0
    # the branch rule is the reference's floating-point comparison of n p and n (1 - p) with 5
    loc, complement = n * p, n * (1.0 - p)
    if approximate and loc > 5.0 and complement > 5.0:
        return oracle.counter_normal(*key) * math.sqrt(loc * (1.0 - p)) + loc, 0, 0
    reverse = p > 0.5
    pr = 1.0 - p if reverse else p   # exact: 1 - p is a double for p in (1/2, 1)
    ties = 0
    for draw in range(64):
        k, tie = inversion(uniform(*key, draw), n, pr)
        ties += tie
        if k >= 0:
            return float(n - k if reverse else k), ties, draw
    raise AssertionError("64 restarts")


def binomial_cases():
    rng = np.random.default_rng(2024)
    cases = []
    for n in (1, 2, 3, 5, 8, 20, 50, 100, 1000, 10_000, 100_000):
        for _ in range(24):
            kind = rng.integers(0, 4)
            if kind == 0:      # inversion from the small tail (n p <= 5 in the approximate mode)
                p = float(rng.uniform(0, min(0.5, 5.0 / n)))
            elif kind == 1:    # reversed tail
                p = 1.0 - float(rng.uniform(0, min(0.5, 5.0 / n)))
            elif kind == 2:    # any p, log-uniform
                p = float(10 ** rng.uniform(-6, 0))
            else:
                p = float(rng.uniform(0, 1))
            cases.append((n, p))
    # around the normal-approximation threshold n p = 5
    for n in (20, 100, 1000):
        for p in (5.0 / n, math.nextafter(5.0 / n, 1), math.nextafter(5.0 / n, 0), 1 - 5.0 / n, 0.999 * 5 / n,
                  1.001 * 5 / n):
            cases.append((n, p))
    return cases


@pytest.mark.parametrize("approximate", [True, False])
def test_binomial_draws_equal_their_definition(approximate):
    """About 3000 draws of counter_binomial over n = 1 .. 100,000 and p in (0, 1), in the
    approximate (PoissonInput) and exact modes, equal the definition draw by draw."""
    ties = restarts = checked = 0
    branches = {"inversion": 0, "reversed": 0, "normal": 0}
    for (n, p), key in zip(binomial_cases() * 10, keys(10_000, 7 + approximate)):
        if not approximate and n * min(p, 1 - p) > 60:
            continue   # exact inversion of large n p: a long search; the approximate mode covers these n
        value, tie, restart = exact_binomial(key, n, p, approximate)
        ties += tie
        restarts += restart > 0
        for shared in (False, True):
            got = oracle.counter_binomial(*key, n, p, approximate, shared=shared)
            if tie:
                assert abs(got - value) <= 1, (key, n, p, got, value)
            else:
                assert got == value, (key, n, p, approximate, shared, got, value)
        checked += 1
        kind = "normal" if value != round(value) else "reversed" if p > 0.5 else "inversion"
        branches[kind] += 1
    assert checked > (2500 if approximate else 1500) and ties <= checked // 1000
    assert branches["inversion"] > 500 and branches["reversed"] > 300
    assert (branches["normal"] > 200) == approximate


def test_binomial_restart_bound():
    """The restart bound of the inversion search, on chosen uniforms near 1 where the exact search
    passes min(n, n p + 10 sqrt(n p q + 1)): the oracle's search returns -1 exactly where the
    definition's does, and the selected k elsewhere."""
    rng = np.random.default_rng(11)
    passed = found = 0
    for n, pr in ((12, 0.01), (40, 0.02), (200, 0.01), (1000, 0.004), (30, 0.2), (100, 0.5), (16, 1e-4)):
        for e in list(range(1, 54)) + list(rng.integers(1, 54, 40)):
            for u in (1.0 - 2.0 ** -int(e), float(rng.uniform(0, 1))):
                k, tie = inversion(u, n, pr)
                if tie:
                    continue
                for shared in (False, True):
                    assert oracle.binomial_search(u, n, pr, shared=shared) == k, (n, pr, u, k)
                passed += k < 0
                found += k >= 0
    assert passed >= 30 and found >= 300


# ------------------------------------------------------------------ poisson
def product_method(key, lam: float):
    """The smallest k with sum_{i <= k} ln u_i <= -lambda; (k, tie)."""
    limit = -mpmath.mpf(lam)
    total = mpmath.mpf(0)
    for k in range(10_000):
        u = uniform(*key, k)
        if u == 0.0:
            return float(k), False
        total += mpmath.log(mpmath.mpf(u))
        if total <= limit:
            return float(k), abs(total - limit) < TIE * (k + 2)
        if abs(total - limit) < TIE * (k + 2):
            return float(k), True
    raise AssertionError("product method did not end")


A_B = {}


def ptrs_constants(lam: float):
    """Hoermann's PTRS constants for lambda (Table 2 of the paper), in exact decimal arithmetic."""
    if lam not in A_B:
        b = mpmath.mpf("0.931") + mpmath.mpf("2.53") * mpmath.sqrt(mpmath.mpf(lam))
        a = mpmath.mpf("-0.059") + mpmath.mpf("0.02483") * b
        inverse_alpha = mpmath.mpf("1.1239") + mpmath.mpf("1.1328") / (b - mpmath.mpf("3.4"))
        squeeze = mpmath.mpf("0.9277") - mpmath.mpf("3.6224") / (b - 2)
        A_B[lam] = (a, b, inverse_alpha, squeeze)
    return A_B[lam]


def ptrs(u: float, v: float, lam: float):
    """One PTRS trial: (candidate or -1, tie)."""
    a, b, inverse_alpha, squeeze = ptrs_constants(lam)
    L = mpmath.mpf(lam)
    U = mpmath.mpf(u) - mpmath.mpf("0.5")
    V = mpmath.mpf(v)
    us = mpmath.mpf("0.5") - abs(U)
    arg = (2 * a / us + b) * U + L + mpmath.mpf("0.43")
    k = mpmath.floor(arg)
    # float evaluation errors scale with the magnitude of the terms: relative 1e-12 of it
    tie = abs(arg - mpmath.nint(arg)) < RELATIVE * max(1, abs(arg))
    tie |= abs(us - mpmath.mpf("0.07")) < TIE or abs(V - squeeze) < TIE
    if us >= mpmath.mpf("0.07") and V <= squeeze:
        return float(k), tie, "squeeze"
    tie |= abs(us - mpmath.mpf("0.013")) < TIE or abs(V - us) < TIE
    if k < 0 or (us < mpmath.mpf("0.013") and V > us):
        return -1.0, tie, "reject"
    left = mpmath.log(V * inverse_alpha / (a / (us * us) + b))
    log_factorial = mpmath.loggamma(k + 1)
    right = -L + k * mpmath.log(L) - log_factorial
    tie |= abs(left - right) < RELATIVE * (1 + L + abs(k * mpmath.log(L)) + log_factorial)
    return (float(k), tie, "test_accept") if left <= right else (-1.0, tie, "test_reject")


def exact_poisson(key, lam: float):
    if lam < 10:
        k, tie = product_method(key, lam)
        return k, int(tie), 0
    ties = 0
    for j in range(0, 200, 2):
        k, tie, _ = ptrs(uniform(*key, j), uniform(*key, j + 1), lam)
        ties += tie
        if k >= 0:
            return k, ties, j // 2
    raise AssertionError("100 PTRS rejections")


def poisson_cases():
    rng = np.random.default_rng(5)
    lams = [float(x) for x in 10 ** rng.uniform(-3, math.log10(9.999), 40)]
    lams += [float(x) for x in 10 ** rng.uniform(1, 6, 60)]
    lams += [1e-9, 0.5, 1.0, 3.0, math.nextafter(10.0, 0), 10.0, 10.5, 50.0, 1e4, 1e9]
    return lams


def test_poisson_draws_equal_their_definition():
    """About 3000 draws of counter_poisson over lambda in [1e-9, 1e9] (the product method below
    10, PTRS above, including draws that a trial's rejection sends to the next pair) equal the
    definition draw by draw."""
    ties = rejected = checked = 0
    for lam, key in zip(poisson_cases() * 28, keys(4000, 3)):
        value, tie, trials = exact_poisson(key, lam)
        ties += tie
        rejected += trials > 0
        for shared in (False, True):
            got = oracle.counter_poisson(*key, lam, shared=shared)
            if tie:
                assert abs(got - value) <= 1, (key, lam, got, value)
            else:
                assert got == value, (key, lam, shared, got, value)
        checked += 1
    assert checked > 2500 and ties <= checked // 1000
    assert rejected > 100


def test_ptrs_trials_equal_their_definition():
    """PTRS trials on chosen uniforms over its branches: the squeeze (us >= 0.07, v <= v_r), the
    rejections (k < 0; us < 0.013 with v > us) and the acceptance test, for lambda from 10 to 1e9."""
    rng = np.random.default_rng(17)
    seen = {"squeeze": 0, "reject": 0, "test_accept": 0, "test_reject": 0}
    for lam in (10.0, 12.5, 30.0, 100.0, 1e3, 1e5, 1e7, 1e9):
        us_edges = np.concatenate([rng.uniform(0, 1, 300), rng.uniform(0, 0.013, 60), 1 - rng.uniform(0, 0.013, 60),
                                   rng.uniform(0.43, 0.57, 60)])
        for u in us_edges:
            v = float(rng.uniform(0, 1))
            k, tie, branch = ptrs(float(u), v, lam)
            if tie:
                continue
            for shared in (False, True):
                assert oracle.ptrs_trial(float(u), v, lam, shared=shared) == k, (u, v, lam, k)
            seen[branch] += 1
    assert all(count >= 30 for count in seen.values()), seen
