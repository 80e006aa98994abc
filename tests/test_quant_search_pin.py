"""Pins the candidate searches inside the Q4_K and Q6_K quantizers of the CPU oracle.

Lattice inputs (test_oracle_pinning.py) are recovered by the searches' first guess, so they never exercise
the stepped candidates.  Here thousands of random sub-blocks go through the oracle's search alone, and an
independent float64 enumeration of the reference's candidate set decides which candidate must win:

* Q4_K (src/torch2vk/quantize/vulkan.py:263-329): weights av_x + |x|, min = min(0, min x); the first guess
  (scale (max - min) / 15, min) and, for s = 0..20, levels at inverse scale (14 + 0.1 s) / (max - min) with a
  weighted least-squares (scale, min), min > 0 refitted with min 0; the lowest weighted error wins, earlier
  candidates winning ties.
* Q6_K (vulkan.py:483-540): weights x^2, levels clamp(round(-(32 + 0.1 s) / max * x), -32, 31) for s = 0 and
  s = -9..-1, 1..9 in that order; the highest (sum w x l)^2 / sum w l^2 wins, earlier candidates winning ties.

The codes are computed with the reference's fp32 operations (which reproduce the oracle's exactly where their
inputs are exact) and the fits and criteria in fp64: a different winner is accepted only where the two
candidates' criteria agree to fp32 rounding, or, for Q4_K, where an error code computed from a fitted min
sits on a half (the fit's last bits, which fp32 and fp64 compute differently, decide it).  Each test also shows that an enumeration with one constant
changed disagrees with the oracle on many sub-blocks, so a wrong constant in the oracle would fail it.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quant

N_Q4, N_Q6 = 3000, 40000


def _inputs(n: int, width: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    q = n // 4
    parts = [rng.standard_normal((q, width)) * 0.02,                               # weights as drawn
             rng.uniform(-1.0, 1.0, (q, width)) + rng.uniform(-0.5, 0.5, (q, 1)),  # shifted
             rng.standard_t(3, (q, width)),                                        # heavy tails
             # all negative: the largest value is near 0 and weighs little, so the finest steps (the
             # largest inverse scales, which clamp it) win too
             -np.abs(rng.standard_normal((n - 3 * q, width)))]
    return np.concatenate(parts).astype(np.float32)


# ------------------------------------------------------------------ Q4_K --

def _levels32(inv: np.ndarray, x: np.ndarray, minimum: np.ndarray, top: int) -> tuple[np.ndarray, np.ndarray]:
    """clamp(floor(inv * (x - min) + 0.5), 0, top) with each operation rounded to fp32, as the reference's
    shader computes the codes, and per row whether any code sits so close to a half that the last bits of min
    or of the product decide it (there fp32 rounding, not the search, picks the candidate)."""
    f = np.float32
    t = (inv.astype(f)[:, None] * (x.astype(f) - minimum.astype(f)[:, None])).astype(f)
    t64 = t.astype(np.float64)
    near_half = np.abs(t64 - np.floor(t64) - 0.5) <= 1e-5 * np.abs(t64) + 1e-6
    inside = (t64 > -0.5) & (t64 < top + 0.5)
    return np.clip(np.floor((t + f(0.5)).astype(f)), 0, top).astype(np.float64), (near_half & inside).any(1)


def q4_k_candidates(x: np.ndarray, start: float = 15.0, base: float = 14.0, step: float = 0.1,
                    n_steps: int = 21) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """(scale, min, error, fragile) [n, 1 + n_steps] of every candidate: codes as fp32 arithmetic makes them,
    the fits and the errors in float64; fragile where a code of the candidate sits on a half."""
    f = np.float32
    x32 = x.astype(f)
    x = x.astype(np.float64)
    n = x.shape[0]
    mn32 = np.minimum(x32.min(1), f(0.0))
    rng32 = (x32.max(1) - mn32).astype(f)
    mn = mn32.astype(np.float64)
    av = np.sqrt((x * x).sum(1) / 32.0)
    w = av[:, None] + np.abs(x)

    def err(scale, minimum, inv):
        lev, frag = _levels32(inv, x32, minimum, 15)
        d = scale[:, None] * lev + minimum[:, None] - x
        return (w * d * d).sum(1), frag

    scales = np.zeros((n, 1 + n_steps))
    mins = np.zeros((n, 1 + n_steps))
    errs = np.full((n, 1 + n_steps), np.inf)
    fragile = np.zeros((n, 1 + n_steps), bool)
    inv0 = (f(start) / rng32).astype(f)
    scales[:, 0], mins[:, 0] = 1.0 / inv0.astype(np.float64), mn
    errs[:, 0], _ = err(scales[:, 0], mins[:, 0], inv0)   # codes from exactly reproduced fp32 values
    sw, sx = w.sum(1), (w * x).sum(1)
    for s in range(n_steps):
        inv = ((f(base) + (f(step) * f(s)).astype(f)).astype(f) / rng32).astype(f)
        lev, _ = _levels32(inv, x32, mn32, 15)   # inv, x and min are the oracle's fp32 values exactly
        sl, sl2, sxl = (w * lev).sum(1), (w * lev * lev).sum(1), (w * lev * x).sum(1)
        det = sw * sl2 - sl * sl
        with np.errstate(divide="ignore", invalid="ignore"):
            sc = (sw * sxl - sx * sl) / det
            m = (sl2 * sx - sl * sxl) / det
            pos = m > 0
            sc = np.where(pos, np.where(sl2 > 0, sxl / sl2, 0.0), sc)
            m = np.where(pos, 0.0, m)
        ok = det > 0
        scales[:, 1 + s] = np.where(ok, sc, 0.0)
        mins[:, 1 + s] = np.where(ok, m, 0.0)
        # the error's codes use the candidate's own fitted min, which fp32 arithmetic computes with other last
        # bits than this float64 fit: a code of it on a half may come out either way
        m32 = np.where(ok, m, 0.0).astype(f)
        e, frag = err(np.where(ok, sc, 0.0), m32.astype(np.float64), inv)
        errs[:, 1 + s] = np.where(ok, e, np.inf)
        fragile[:, 1 + s] = frag & ok
    return scales, mins, errs, fragile


def _q4_k_unexplained(x, got_scale, got_min, **perturb) -> int:
    scales, mins, errs, fragile = q4_k_candidates(x, **perturb)
    best = np.argmin(errs, axis=1)  # first minimum: earlier candidates win ties
    cand_scale = np.maximum(scales, 0.0)
    cand_min = np.maximum(-mins, 0.0)
    tol = lambda a: 2e-5 * np.abs(a) + 1e-12  # noqa: E731  fp32 rounding of the oracle's results
    rows = np.arange(x.shape[0])
    same = (np.abs(cand_scale[rows, best] - got_scale) <= tol(got_scale)) & \
           (np.abs(cand_min[rows, best] - got_min) <= tol(got_min))
    unexplained = 0
    for i in np.flatnonzero(~same):
        # the oracle kept another candidate: allowed only if its error ties the best one to fp32 rounding
        match = np.flatnonzero((np.abs(cand_scale[i] - got_scale[i]) <= tol(got_scale[i])) &
                               (np.abs(cand_min[i] - got_min[i]) <= tol(got_min[i])))
        tie = match.size and np.any(errs[i, match] <= errs[i, best[i]] * (1 + 1e-5) + 1e-12)
        rounding = match.size and (fragile[i, best[i]] or np.any(fragile[i, match]))
        if not (tie or rounding):
            unexplained += 1
    return unexplained


def test_q4_k_search_keeps_the_reference_candidate():
    x = _inputs(N_Q4, 32, 1)
    got_scale, got_min = quant.q4_k_subblock_search(x)
    _, _, errs, fragile = q4_k_candidates(x)
    print(f"sub-blocks with a candidate code on a half: {int(fragile.any(1).sum())} of {N_Q4}")
    winners = np.bincount(np.argmin(errs, axis=1), minlength=22)
    print(f"winning Q4_K candidate (0 = first guess, 1 + s = step s): {winners.tolist()}")
    # the inputs exercise the search: the first guess and every step win somewhere
    assert np.all(winners > 0)
    assert _q4_k_unexplained(x, got_scale, got_min) == 0


@pytest.mark.parametrize("perturb", [dict(step=0.11), dict(base=14.5), dict(n_steps=20), dict(start=15.5)])
def test_q4_k_search_pin_rejects_other_constants(perturb):
    x = _inputs(N_Q4, 32, 1)
    got_scale, got_min = quant.q4_k_subblock_search(x)
    bad = _q4_k_unexplained(x, got_scale, got_min, **perturb)
    print(f"{perturb}: {bad} of {N_Q4} sub-blocks disagree")
    assert bad > 0  # the acceptance test above, which allows none, would fail


# ------------------------------------------------------------------ Q6_K --

def q6_k_candidates(x: np.ndarray, base: float = 32.0, step: float = 0.1, span: int = 9):
    """(scale, criterion, levels) of the candidates in the reference's order: levels from the same fp32
    operations as the reference's shader (inverse scale, product, round half to even), which reproduces the
    oracle's levels exactly; scale and criterion in float64."""
    f = np.float32
    x32 = x.astype(f)
    x = x.astype(np.float64)
    idx = np.argmax(np.abs(x32), axis=1)  # first maximum of |x|, as the strict > scan keeps
    mx = x32[np.arange(x.shape[0]), idx]
    w = x * x
    order = [0] + list(range(-span, 0)) + list(range(1, span + 1))
    scales, crit, levels = [], [], []
    for s in order:
        numer = (f(base) + (f(step) * f(s)).astype(f)).astype(f) if s else f(base)
        inv = (-numer / mx).astype(f)
        lev = np.clip(np.rint((inv[:, None] * x32).astype(f)), -32, 31).astype(np.float64)
        sl2 = (w * lev * lev).sum(1)
        slx = (w * x * lev).sum(1)
        with np.errstate(divide="ignore", invalid="ignore"):
            scales.append(np.where(sl2 > 0, slx / sl2, 0.0))
            crit.append(np.where(sl2 > 0, slx * slx / sl2, -np.inf))
        levels.append(lev)
    return np.stack(scales, 1), np.stack(crit, 1), np.stack(levels, 1)


def _q6_k_unexplained(x, got_scale, got_levels, **perturb) -> int:
    scales, crit, levels = q6_k_candidates(x, **perturb)
    best = np.argmax(crit, axis=1)  # first maximum: earlier candidates win ties
    rows = np.arange(x.shape[0])
    tol = 2e-5 * np.abs(got_scale) + 1e-12
    same = (np.abs(scales[rows, best] - got_scale) <= tol) & \
           np.all(levels[rows, best] + 32 == got_levels, axis=1)
    unexplained = 0
    for i in np.flatnonzero(~same):
        match = np.flatnonzero(np.all(levels[i] + 32 == got_levels[i], axis=1))
        # the oracle kept other levels: allowed only if their criterion ties the best one to fp32 rounding
        if not (match.size and np.any(crit[i, match] >= crit[i, best[i]] * (1 - 1e-5))):
            unexplained += 1
    return unexplained


def _q6_k_inputs(n: int, seed: int) -> np.ndarray:
    """Random sub-blocks, plus sub-blocks whose other values lie within a fraction of the largest one (same sign):
    there the levels of the near-maximal values move between steps and the steps down to s = -9 and up to s = 5
    win (larger steps only map those values further past the clamped maximum)."""
    rng = np.random.default_rng(seed)
    q = n // 4
    parts = [_inputs(q, 16, seed)]
    for lo in (0.5, 0.8, 0.95):
        m = q if lo != 0.95 else n - 3 * q
        x = -rng.uniform(lo, 1.0, (m, 16)) * rng.uniform(0.01, 2.0, (m, 1))
        x[np.arange(m), rng.integers(0, 16, m)] = x.min(1)   # no second value of the same magnitude
        parts.append(x * rng.choice([-1.0, 1.0], (m, 1)))
    return np.concatenate(parts).astype(np.float32)


def test_q6_k_search_keeps_the_reference_candidate():
    x = _q6_k_inputs(N_Q6, 2)
    got_scale, got_levels = quant.q6_k_subblock_search(x)
    _, crit, _ = q6_k_candidates(x)
    winners = np.bincount(np.argmax(crit, axis=1), minlength=19)
    print(f"winning Q6_K candidate (0 = s 0, then s = -9..-1, 1..9): {winners.tolist()}")
    # s = 0, -9..-1 and 1..5 each win somewhere; s = 6..9 won on none of 2e5 sampled sub-blocks of these
    # families, so sampling cannot pin them (nor can they change a quantized block where they never win)
    assert np.all(winners[:15] > 0)
    assert _q6_k_unexplained(x, got_scale, got_levels) == 0


@pytest.mark.parametrize("perturb", [dict(step=0.11), dict(base=32.5), dict(span=8)])
def test_q6_k_search_pin_rejects_other_constants(perturb):
    x = _q6_k_inputs(N_Q6, 2)
    got_scale, got_levels = quant.q6_k_subblock_search(x)
    bad = _q6_k_unexplained(x, got_scale, got_levels, **perturb)
    print(f"{perturb}: {bad} of {N_Q6} sub-blocks disagree")
    assert bad > 0  # the acceptance test above, which allows none, would fail
