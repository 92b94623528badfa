"""The sampler's threshold search (CPU): the reference's 32 f32 bisection steps on [0, 1]
(sample.wgsl:241-261: mid = (lo + hi) * 0.5, mass(p >= mid) < topP ? hi = mid : lo = mid) end on
the same lo as the same steps driven by one value, p* = the largest probability whose upper mass
mass(p >= p*) reaches topP (mid > p* exactly when mass(p >= mid) < topP). The GPU finds p* by radix
selection over the bits of p and replays the steps from it; this checks the equivalence on
distributions the sampler meets (flat random-init logits, peaked, ties, a few survivors) and the
topP edges (0, 1 - 2^-24), with masses in the GPU's integer fixed point (p * 2^52)."""

import numpy as np
import pytest

FIX = 2.0 ** 52


def fix(p):
    return np.rint(p.astype(np.float64) * FIX).astype(np.uint64)


def bisection(p, top_p):
    """The reference's 32 steps with exact (integer) masses."""
    m = fix(p)
    lo, hi = np.float32(0), np.float32(1)
    need = float(np.float32(top_p)) * FIX
    for _ in range(32):
        mid = np.float32((lo + hi) * np.float32(0.5))
        mass = int(m[p >= mid].sum(dtype=np.uint64))
        if mass < need:
            hi = mid
        else:
            lo = mid
    return lo


def from_pstar(p, top_p):
    """p* from the probabilities sorted in descending order (by radix selection on the GPU), then
    the same 32 steps comparing each mid with p*."""
    need = float(np.float32(top_p)) * FIX
    if need <= 0:
        pstar = np.float32(np.inf)
    else:
        vals = np.unique(p)[::-1]  # distinct values, descending
        m = fix(p)
        pstar = None
        for v in vals:
            if float(int(m[p >= v].sum(dtype=np.uint64))) >= need:
                pstar = v
                break
        if pstar is None:  # the whole mass short of topP: threshold 0
            return np.float32(0)
    lo, hi = np.float32(0), np.float32(1)
    for _ in range(32):
        mid = np.float32((lo + hi) * np.float32(0.5))
        if mid > pstar:
            hi = mid
        else:
            lo = mid
    return lo


def softmax32(logits, t):
    z = (logits / np.float32(t)).astype(np.float32)
    e = np.exp((z - z.max()).astype(np.float32)).astype(np.float32)
    return (e / np.float32(e.astype(np.float64).sum())).astype(np.float32)


CASES = {
    "flat": lambda r: softmax32(r.standard_normal(4096).astype(np.float32) * np.float32(0.05), 0.7),
    "peaked": lambda r: softmax32(r.standard_normal(4096).astype(np.float32) * np.float32(4.0), 0.7),
    "ties": lambda r: softmax32(np.repeat(r.standard_normal(64).astype(np.float32), 64), 1.0),
    "few": lambda r: softmax32(np.concatenate([np.full(4090, -30, np.float32), r.standard_normal(6).astype(np.float32) * 3]), 1.0),
    "two": lambda r: np.array([0.75, 0.25], np.float32),
}


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("top_p", [0.0, 0.1, 0.5, 0.9, 0.95, 1.0 - 2.0 ** -24])
def test_bisection_follows_pstar(case, top_p):
    p = CASES[case](np.random.default_rng(11))
    assert bisection(p, top_p) == from_pstar(p, top_p)


def test_kept_set_is_the_nucleus():
    """At the threshold both searches end on, the kept mass reaches topP and dropping the smallest
    kept probability would fall short of it (the nucleus)."""
    p = CASES["peaked"](np.random.default_rng(5))
    for top_p in (0.5, 0.9):
        thr = from_pstar(p, top_p)
        kept = np.sort(p[p >= thr])
        assert kept.astype(np.float64).sum() >= top_p - 1e-6
        assert kept[1:].astype(np.float64).sum() < top_p + 1e-6
