"""GPU parity: the HIP sampler against the CPU oracle on the same bytes.

Configs 1-3 run at their full BASELINE sizes; configs 4-5 (the full-vocab
path) at reduced batch.
"""
import numpy as np
import pytest

from oracle import oracle
from parity_util import compare, run_both
from scriptonait_amd.workloads import PARAMS_DTYPE, make_params, make_workload

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_configs_full_size(sampler, cfg):
    w = make_workload(cfg)
    g, o = run_both(sampler, w)
    s = compare(g, o, w.name)
    print(w.name, s, flush=True)


@pytest.mark.parametrize("cfg,B", [(4, 16), (5, 8)])
def test_full_vocab_configs_reduced_batch(sampler, cfg, B):
    w = make_workload(cfg, B=B)
    g, o = run_both(sampler, w)
    s = compare(g, o, w.name)
    print(w.name, s, flush=True)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_other_data_seeds_config3(sampler, seed):
    w = make_workload(3, data_seed=seed, B=64)
    g, o = run_both(sampler, w)
    compare(g, o, f"config3 seed {seed}")


def test_greedy_rows(sampler):
    w = make_workload(3, B=32)
    prm = make_params(0.0, 64, 0.95, 0.05, 1.15)
    g, o = run_both(sampler, w, params=prm)
    assert np.array_equal(g.ids, o.ids)
    assert np.array_equal(g.rng_state, w.rng_seeds), "greedy rows must not advance the RNG"


def test_per_row_mixed_params(sampler):
    w = make_workload(2, B=48)
    prm = np.zeros(48, dtype=PARAMS_DTYPE)
    for b in range(48):
        kind = b % 6
        prm[b] = [(0.0, 50, 0.9, 0.1, 1.2), (1.0, 50, 0.9, 0.1, 1.2), (0.7, 1, 1.0, 0.0, 1.0),
                  (1.3, 0, 0.9, 0.0, 1.1), (1.0, 8192, 1.0, 0.2, 1.0), (0.5, 1000, 0.5, 0.0, 0.8)][kind]
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, "mixed per-row params")


@pytest.mark.parametrize("B", [2048, 2049])
def test_mixed_classes_on_both_sides_of_the_host_class_table(sampler, B):
    """A call of up to 2048 rows carries each row's class in the kernel
    arguments (its launches skip other classes' rows before any load); a
    larger one finds the class from the row's parameters. Both must sample
    every row once, by the path of its own class."""
    w = make_workload(2, B=B)
    prm = np.zeros(B, dtype=PARAMS_DTYPE)
    kinds = [(0.0, 50, 0.9, 0.1, 1.2), (1.0, 50, 0.9, 0.1, 1.2), (1.3, 0, 0.9, 0.0, 1.1),
             (0.5, 5000, 0.5, 0.0, 1.0)]  # greedy, top-k, whole vocabulary, K above the register path
    order = np.random.default_rng(B).integers(0, len(kinds), size=B)
    for b in range(B):
        prm[b] = kinds[order[b]]
    g, o = run_both(sampler, w, params=prm, want_probs=False)
    s = compare(g, o, f"mixed classes B={B}", probs=False)
    assert s["mismatches"] == 0, s


def test_allowed_mask(sampler):
    w = make_workload(2, B=16)
    allowed = np.ones(w.V - 100, dtype=np.uint8)  # ids past the mask stay allowed
    allowed[::3] = 0
    allowed[258] = 0  # EOS is always allowed
    g, o = run_both(sampler, w, allowed=allowed)
    compare(g, o, "allowed mask")


@pytest.mark.parametrize("V", [1, 5, 7, 64, 257, 1000, 4097, 12345])
def test_odd_vocab_sizes(sampler, V):
    w = make_workload(3, B=6, V=V)
    for k in (1, 3, 40):
        prm = make_params(0.8, k, 0.95, 0.05, 1.1)
        g, o = run_both(sampler, w, params=prm)
        compare(g, o, f"V={V} k={k}")


def test_all_masked_row_is_degenerate(sampler):
    V = 300
    logits = np.full((2, V), -np.inf, dtype=np.float32)
    prm = make_params(0.9, 40, 0.95, 0.0, 1.1)
    seeds = np.array([5, 6], dtype=np.uint64)
    g = sampler.sample_host(logits, prm, seeds)
    assert list(g.ids) == [0, 0]
    assert np.array_equal(g.rng_state, seeds), "degenerate rows must not draw"


def test_ties_resolve_by_smallest_id(sampler):
    V = 2048
    logits = np.zeros((4, V), dtype=np.float32)  # every value tied
    prm = make_params(1.0, 5, 1.0, 0.0, 1.0)
    seeds = np.arange(4, dtype=np.uint64)
    from oracle import oracle

    g = sampler.sample_host(logits, prm, seeds, want_probs=True)
    o = oracle.sample_batch(logits, prm, seeds, want_probs=True)
    assert np.array_equal(g.ids, o.ids)
    assert set(g.ids.tolist()) <= {0, 1, 2, 3, 4}


@pytest.mark.parametrize("T", [0.05, 0.3, 0.7, 1.7, 8.0, 30.0, 100.0])
def test_temperatures_merge_ties(sampler, T):
    """Division by T can merge distinct logits into equal values, which the
    reference then orders by id; small and large T stress that boundary."""
    w = make_workload(3, B=32)
    prm = make_params(T, 64, 0.95, 0.05, 1.15)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, f"T={T}")


def test_quantized_logits_many_ties(sampler):
    """Logits on a coarse grid: thousands of exact ties around the top-k cut."""
    w = make_workload(3, B=16)
    w.logits[:] = np.round(w.logits * 4.0) / 4.0
    for k in (1, 16, 64, 500):
        prm = make_params(0.9, k, 0.97, 0.01, 1.1)
        g, o = run_both(sampler, w, params=prm)
        compare(g, o, f"quantized k={k}")


def test_long_history_with_repeats(sampler):
    """History longer than 2048 ids (loaded in the loop), heavy repeats."""
    w = make_workload(3, B=8)
    H = 5000
    rs = np.random.default_rng(7)
    hist = rs.integers(0, 50, size=8 * H).astype(np.uint32)  # ids repeat ~100 times
    hist[::7] = rs.integers(0, w.V + 100, size=hist[::7].size)  # some ids >= V (ignored)
    offs = (np.arange(9) * H).astype(np.uint32)
    g = sampler.sample_host(w.logits, w.params, w.rng_seeds, hist, offs, V=w.V, want_probs=True)
    from oracle import oracle

    o = oracle.sample_batch(w.logits, w.params, w.rng_seeds, hist, offs, V=w.V, want_probs=True)
    compare(g, o, "long history")


_GOLDEN = 0x9E3779B97F4A7C15
_M1, _M2 = 0xBF58476D1CE4E5B9, 0x94D049BB133111EB
_MASK = (1 << 64) - 1


def _seed_for_draw(m24: int) -> int:
    """A SplitMix64 seed whose first f32 draw (rng.rs:24-34: the top 24 bits
    of the first output, times 2^-24) is exactly m24 * 2^-24. The output mix
    is a bijection; this runs it backwards."""
    def unxorshift(z, s):
        x = z
        for _ in range(64 // s + 1):
            x = z ^ (x >> s)
        return x & _MASK
    z = (m24 << 40) & _MASK
    z = unxorshift(z, 31)
    z = (z * pow(_M2, -1, 1 << 64)) & _MASK
    z = unxorshift(z, 27)
    z = (z * pow(_M1, -1, 1 << 64)) & _MASK
    z = unxorshift(z, 30)
    return (z - _GOLDEN) & _MASK


@pytest.mark.parametrize("V", [4096, 32000])
def test_exact_ties_in_the_top_p_and_draw_folds(sampler, V):
    """64 equal top values give p_i = 1/64 and exact cumulative sums: top-p
    cut-offs that land exactly on a cumulative value and draws that land
    exactly on a walk boundary, where only an exact replay of the f32 folds
    decides (generate.rs:397-419)."""
    from oracle import oracle
    from scriptonait_amd.workloads import splitmix64_outputs

    assert splitmix64_outputs(_seed_for_draw(0x400000), 1)[0] >> np.uint64(40) == 0x400000
    rs = np.random.default_rng(5)
    B = 96
    logits = (rs.standard_normal((B, V)) - 20.0).astype(np.float32)
    for b in range(B):
        logits[b, rs.choice(V, 64, replace=False)] = 5.0
    prm = np.zeros(B, dtype=PARAMS_DTYPE)
    seeds = np.zeros(B, dtype=np.uint64)
    for b in range(B):
        top_p = [0.5, 0.25, 1.0, 0.75 + 2.0 ** -20][b % 4]
        prm[b] = (1.0, 64, top_p, [0.0, 0.5][b % 2], 1.0)
        seeds[b] = _seed_for_draw((b % 32) << 19)  # u = (b % 32) / 32: exact walk boundaries
    g = sampler.sample_host(logits, prm, seeds, want_probs=True)
    o = oracle.sample_batch(logits, prm, seeds, want_probs=True)
    assert np.array_equal(g.ids, o.ids), np.nonzero(g.ids != o.ids)[0]
    assert np.array_equal(g.kept, o.kept)
    assert np.array_equal(g.rng_state, o.rng_state)


@pytest.mark.parametrize("V,temp,k", [(32000, 0.7, 64), (32000, 0.0, 64), (12345, 1.0, 40), (4099, 0.0, 8),
                                      (32000, 1.0, 700)])
def test_history_of_each_rows_top_candidates(sampler, V, temp, k):
    """The history holds each row's own highest logits, 1-4 times each, plus
    random ids (a long generation's window: what was drawn is what ranks
    high). The penalty pushes most of the raw top below the speculative
    threshold, so the register path must take its proven threshold, and
    greedy rows their bounded penalty pass; every row must still match the
    oracle and none may be handed to the sorting path."""
    B = 24
    w = make_workload(3, B=B, V=V)
    rs = np.random.default_rng(V + k)
    rows = []
    for b in range(B):
        top = np.argsort(-w.logits[b, :V], kind="stable")[: 3 * k]
        reps = rs.integers(1, 5, size=top.size)
        ids = np.concatenate([np.repeat(top, reps), rs.integers(0, V, size=2000)]).astype(np.uint32)
        rows.append(rs.permutation(ids))
    offs = np.concatenate([[0], np.cumsum([r.size for r in rows])]).astype(np.uint32)
    hist = np.concatenate(rows)
    prm = make_params(temp, k, 0.95, 0.02, 1.3)
    sampler.status()  # clears the hand-over count
    g = sampler.sample_host(w.logits, prm, w.rng_seeds, hist, offs, V=V, want_probs=temp > 0)
    handovers = sampler.status().handovers
    o = oracle.sample_batch(w.logits, prm, w.rng_seeds, hist, offs, V=V, want_probs=temp > 0, threads=8)
    if temp > 0:
        compare(g, o, f"top-candidate history V={V} k={k}")
    else:
        assert np.array_equal(g.ids, o.ids)
    assert handovers == 0
