"""The error bounds behind the fast tail's top-p and draw decisions.

The gfx950 tail (scriptonait_amd/csrc/draw_tail.h, draw_tail_bcast) decides
top-p (generate.rs:397-409) and the inverse-CDF walk (generate.rs:412-419)
from f64 prefix sums of the probabilities, with bounds on how far the
reference's f32 left folds can drift from them:

    |c_i - P_i| <= B_i = i * hulp(P_i (1 + 2^-17))
    r_i in [u lo(c_s) - P_{i-1} - G_i, u hi(c_s) - P_{i-1} + G_i],
    G_i = (i + 1) * hulp(u hi(c_s) (1 + 2^-16))

(hulp = half an f32 ulp in the binade of its argument). A decision is taken
only when the interval settles it; near ties replay the folds exactly. This
CPU test restates those decision rules in numpy and checks them against the
exact f32 folds by brute force, on random rows and on rows built to put
top_p and the draw exactly on a fold value (where the rules must refuse to
decide): a bound that is too tight fails here as a wrong decision.
"""
import numpy as np

f32 = np.float32


def exact_folds(p, keep, top_p, u):
    """generate.rs:397-419 on f32 values, one element at a time."""
    stop = keep
    if top_p < 1.0:
        c = f32(0.0)
        for i in range(keep):
            c = f32(c + p[i])
            if c >= f32(top_p):
                stop = i + 1
                break
    total = f32(0.0)
    for i in range(stop):
        total = f32(total + p[i])
    r = f32(f32(u) * total)
    for i in range(stop):
        if r < p[i]:
            return stop, i
        r = f32(r - p[i])
    return stop, stop - 1


def hulp(x):
    e = np.frexp(np.maximum(x, 2.0 ** -60))[1]
    return np.ldexp(1.0, e - 25)


def certified(p, keep, top_p, u):
    """The kernel's rules; None where it falls back to the exact folds."""
    lane = np.arange(64)
    pd = np.zeros(64)
    pd[:keep] = p[:keep]
    Pi = np.cumsum(pd)
    Bi = lane * hulp(Pi * (1 + 2.0 ** -17)) + 2.0 ** -45 * Pi
    stop = keep
    if top_p < 1.0:
        tpd = float(f32(top_p))
        poss = (lane < keep) & ~(Pi + Bi < tpd)
        sure = (lane < keep) & (Pi - Bi >= tpd)
        if poss.any():
            i = int(np.argmax(poss))
            if not sure[i]:
                return None
            stop = i + 1
    s = stop - 1
    U = float(f32(u))
    lo0, hi0 = U * (Pi[s] - Bi[s]), U * (Pi[s] + Bi[s])
    Pprev = Pi - pd
    Gi = (lane + 1) * hulp(hi0 * (1 + 2.0 ** -16)) + 2.0 ** -45 * (hi0 + Pprev)
    pdd = np.zeros(64)
    pdd[:len(p)] = p
    poss = (lane < stop) & ~(lo0 - Pprev - Gi >= pdd)
    sure = (lane < stop) & (hi0 - Pprev + Gi < pdd)
    if not poss.any():
        return stop, stop - 1
    i = int(np.argmax(poss))
    return (stop, i) if sure[i] else None


def _row(rng, kind, n=64):
    if kind == 0:
        w = rng.normal(0, 0.5, n) / 0.7
    elif kind == 1:
        w = rng.normal(0, 4, n) / 0.7
    elif kind == 2:
        w = rng.gumbel(size=n)
    else:
        w = rng.uniform(-30, 0, n)
    w = np.sort(w.astype(f32))[::-1]
    e = np.exp((w - w[0]).astype(np.float64)).astype(f32)
    s = f32(0.0)
    for x in e:
        s = f32(s + x)
    return (e / s).astype(f32)


def _keep(p, min_p):
    if min_p <= 0:
        return len(p)
    bad = np.nonzero(~(p >= f32(f32(min_p) * p[0])))[0]
    return max(1, int(bad[0])) if bad.size else len(p)


def test_decisions_match_exact_folds_on_random_rows():
    rng = np.random.default_rng(11)
    decided = 0
    for t in range(4000):
        p = _row(rng, t % 4)
        keep = _keep(p, [0.0, 0.05][t % 2])
        top_p = [0.95, 0.9, 1.0, 0.5][t % 4]
        u = f32(rng.integers(0, 1 << 24) * 2.0 ** -24)
        got = certified(p, keep, top_p, u)
        if got is not None:
            decided += 1
            assert got == exact_folds(p, keep, top_p, u), (t, keep, top_p, u)
    assert decided > 3900  # near ties are rare


def test_decisions_refuse_exact_ties():
    """top_p equal to (or one ulp from) an f32 cumulative value and draws
    that land on a walk boundary: every decision taken must still be right."""
    rng = np.random.default_rng(12)
    for t in range(4000):
        p = _row(rng, t % 4)
        keep = _keep(p, [0.0, 0.05][t % 2])
        c, cs = f32(0.0), []
        for i in range(keep):
            c = f32(c + p[i])
            cs.append(c)
        j = int(rng.integers(0, keep))
        top_p = float(np.nextafter(cs[j], [f32(-1), f32(2), cs[j]][t % 3]))
        if top_p >= 1.0:
            top_p = 0.9
        u = f32(rng.integers(0, 1 << 24) * 2.0 ** -24)
        if t % 5 == 0:
            stop, _ = exact_folds(p, keep, top_p, 0.5)
            tot = f32(0.0)
            for i in range(stop):
                tot = f32(tot + p[i])
            k = int(rng.integers(0, stop))
            pre = f32(0.0)
            for i in range(k):
                pre = f32(pre + p[i])
            u = f32(pre / tot)
        got = certified(p, keep, top_p, u)
        if got is not None:
            assert got == exact_folds(p, keep, top_p, u), (t, keep, top_p, u)
