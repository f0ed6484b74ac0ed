"""Pinning the CPU oracle (oracle/sampler_oracle.cpp) on the CPU.

Checks, in order of strength:
  * SplitMix64 against Vigna's published output for seed 0 and against the
    closed form state_n = seed + n * 0x9E3779B97F4A7C15;
  * the reference's own sampler and PRNG property tests
    (crates/llm-core/src/generate.rs:550-692, crates/llm-core/src/rng.rs:48-91);
  * closed forms: top_k = 1 and greedy give the argmax; flat logits without
    truncation make the drawn index floor(u * n);
  * brute force over all 2^24 draws of a tiny row: each id's share of draws
    is its f32 probability mass, and the oracle's draw for a seed is the
    table entry at that seed's u;
  * an independent pure-Python restatement (tests/pyref.py) on random rows.
"""
import numpy as np
import pytest

from oracle import oracle
from pyref import PyRng, sample_with as py_sample_with
from scriptonait_amd.workloads import PARAMS_DTYPE, make_params, splitmix64_outputs

GOLD = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def one(logits, T=0.9, k=40, p=0.95, mp=0.0, rp=1.1, recent=(), seed=0, allowed=None):
    logits = np.asarray(logits, dtype=np.float32)
    prm = make_params(T, k, p, mp, rp)
    h = np.asarray(recent, dtype=np.uint32)
    offs = np.array([0, h.size], dtype=np.uint32)
    r = oracle.sample_batch(logits[None, :], prm, np.array([seed], dtype=np.uint64),
                            h if h.size else None, offs if h.size else None, allowed=allowed)
    return int(r.ids[0]), int(r.rng_state[0])


# --- SplitMix64 -------------------------------------------------------------
def test_splitmix64_published_output_seed0():
    # Vigna's splitmix64.c, x = 0: the first three outputs.
    s = 0
    outs = []
    for _ in range(3):
        o, s = oracle.splitmix64_next(s)
        outs.append(o)
    assert outs == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_splitmix64_state_closed_form():
    for seed in (0, 1, 42, M64, 0x123456789ABCDEF):
        s = seed
        for n in range(1, 50):
            _, s = oracle.splitmix64_next(s)
            assert s == (seed + n * GOLD) & M64


def test_next_f32_is_top24_bits_over_2_24():
    for seed in (0, 7, 42, 999):
        out, _ = oracle.splitmix64_next(seed)
        f, _ = oracle.next_f32(seed)
        assert f == (out >> 40) / float(1 << 24)
        assert 0.0 <= f < 1.0
    f0, _ = oracle.next_f32(0)
    assert f0 == 14819496 / 2 ** 24  # 0xe220a8 / 2^24


def test_numpy_stream_matches_oracle():
    seed = 0xDEADBEEF
    z = splitmix64_outputs(seed, 20)
    s = seed
    for k in range(20):
        o, s = oracle.splitmix64_next(s)
        assert int(z[k]) == o


# rng.rs:48-91 (ported)
def test_rng_deterministic_for_same_seed():
    a, b = 7, 7
    for _ in range(10):
        oa, a = oracle.splitmix64_next(a)
        ob, b = oracle.splitmix64_next(b)
        assert oa == ob


def test_rng_different_seeds_diverge():
    assert oracle.splitmix64_next(1)[0] != oracle.splitmix64_next(2)[0]


def test_rng_next_f32_in_unit_interval():
    s = 999
    for _ in range(1000):
        f, s = oracle.next_f32(s)
        assert 0.0 <= f < 1.0


# --- generate.rs:550-692, ported -------------------------------------------
def test_top_k_restricts_the_choice_to_the_k_best():
    for seed in range(50):
        picked, _ = one([0.0, 5.0, 0.0, 9.0, 0.0], T=5.0, k=2, p=1.0, rp=1.0, seed=seed)
        assert picked in (3, 1)


def test_top_p_keeps_the_nucleus():
    for seed in range(20):
        assert one([20.0, 0.0, 0.0, 0.0], T=1.0, k=0, p=0.9, rp=1.0, seed=seed)[0] == 0


def test_repetition_penalty_pushes_recent_tokens_down():
    assert one([2.0, 1.9, 0.0], T=0.0, rp=1.5, recent=[], seed=1)[0] == 0
    assert one([2.0, 1.9, 0.0], T=0.0, rp=1.5, recent=[0], seed=1)[0] == 1


def test_min_p_cuts_the_tail_of_a_confident_step():
    s = 1
    for _ in range(64):
        picked, s = one([6.0] + [0.0] * 7, T=1.0, k=0, p=1.0, mp=0.1, rp=1.0, seed=s)
        assert picked == 0


def test_min_p_keeps_the_field_when_the_model_is_unsure():
    s = 2
    seen = set()
    for _ in range(500):
        picked, s = one([0.10, 0.05, 0.0, -0.05, -0.10], T=1.0, k=0, p=1.0, mp=0.1, rp=1.0, seed=s)
        seen.add(picked)
    assert seen == {0, 1, 2, 3, 4}


def test_min_p_always_leaves_a_candidate():
    assert one([1.0, 0.9, 0.8], T=1.0, k=0, p=1.0, mp=5.0, rp=1.0, seed=3)[0] == 0


def test_min_p_is_off_unless_asked_for():
    from scriptonait_amd.sampler import SamplingConfig

    assert SamplingConfig().min_p == 0.0


# --- closed forms -----------------------------------------------------------
def test_top_k_one_and_greedy_give_the_argmax():
    rs = np.random.default_rng(0)
    for _ in range(50):
        x = rs.normal(size=97).astype(np.float32)
        am = int(np.argmax(x))
        assert one(x, T=0.0, rp=1.0)[0] == am
        assert one(x, T=0.7, k=1, p=1.0, rp=1.0, seed=int(rs.integers(1 << 62)))[0] == am


def test_greedy_does_not_advance_the_rng():
    _, s = one([1.0, 2.0], T=0.0, seed=77)
    assert s == 77


def test_flat_logits_draw_index_is_floor_u_times_n():
    # p_i = 1/n exactly representable for n a power of two; r = u and each
    # step subtracts 1/n exactly, so the walk stops at floor(u * n).
    for n in (2, 4, 8, 16, 64):
        for seed in range(40):
            u, _ = oracle.next_f32(seed)
            picked, _ = one(np.zeros(n), T=1.0, k=0, p=1.0, rp=1.0, seed=seed)
            assert picked == int(u * n)


def test_degenerate_rows_take_the_fallback_without_drawing():
    ninf = -np.inf
    picked, s = one([ninf, ninf, ninf], T=1.0, k=0, p=1.0, rp=1.0, seed=5)
    assert (picked, s) == (0, 5)
    picked, s = one([], T=1.0, k=0, p=1.0, rp=1.0, seed=5)
    assert (picked, s) == (0, 5)


def test_allowed_mask_keeps_eos_and_ids_past_its_end():
    x = np.zeros(300, dtype=np.float32)
    x[258] = 5.0  # EOS is always allowed
    x[299] = 4.0  # past the end of the mask: allowed
    allowed = np.zeros(280, dtype=np.uint8)
    assert one(x, T=0.0, rp=1.0, allowed=allowed)[0] == 258
    x[258] = 0.0
    assert one(x, T=0.0, rp=1.0, allowed=allowed)[0] == 299


def test_penalty_applies_once_per_occurrence_and_ignores_out_of_range_ids():
    # 3.0 / 1.5^2 = 1.333 < 1.5: two occurrences push token 0 below token 1.
    assert one([3.0, 1.5], T=0.0, rp=1.5, recent=[0])[0] == 0
    assert one([3.0, 1.5], T=0.0, rp=1.5, recent=[0, 0])[0] == 1
    assert one([3.0, 1.5], T=0.0, rp=1.5, recent=[0, 7, 99])[0] == 0
    # negative logits are multiplied: -1 * 1.5 = -1.5 < -1.2
    assert one([-1.0, -1.2], T=0.0, rp=1.5, recent=[0])[0] == 1


# --- brute force over every draw --------------------------------------------
def test_all_2_24_draws_of_a_tiny_row():
    """For every possible u = m / 2^24 the walk is replayed in float32
    (vectorized over u); each id's share of the 2^24 draws must equal its
    mass to within the 2^-24 draw granularity, and the oracle's pick for a
    seed must be the table entry at that seed's u."""
    logits = np.array([1.3, 0.2, 0.9, -0.4, 0.9, 2.1], dtype=np.float32)
    T, k, p, mp = 0.8, 5, 0.97, 0.05
    ref_id, kept = py_sample_with(logits, T, k, p, mp, 1.0, [], PyRng(0))
    ids = list(kept.keys())
    probs = np.array([kept[i] for i in ids], dtype=np.float32)
    total = np.float32(0)
    for q in probs:
        total = np.float32(total + q)
    u = (np.arange(1 << 24, dtype=np.float64) / (1 << 24)).astype(np.float32)
    r = (u * total).astype(np.float32)
    choice = np.full(u.size, len(ids) - 1, dtype=np.int64)
    done = np.zeros(u.size, dtype=bool)
    for i, q in enumerate(probs):
        hit = (~done) & (r < q)
        choice[hit] = i
        done |= hit
        r = (r - q).astype(np.float32)
    counts = np.bincount(choice, minlength=len(ids)) / float(1 << 24)
    assert np.all(np.abs(counts - probs / total) < 4.0 / (1 << 24) + 1e-7)
    assert np.all(np.diff(choice) >= 0)  # inverse CDF: monotone in u
    for seed in range(200):
        uu, _ = oracle.next_f32(seed)
        picked, _ = one(logits, T=T, k=k, p=p, mp=mp, rp=1.0, seed=seed)
        assert picked == ids[choice[int(round(uu * (1 << 24)))]]


# --- independent restatement ------------------------------------------------
@pytest.mark.parametrize("case", range(60))
def test_oracle_matches_pure_python_restatement(case):
    rs = np.random.default_rng(1000 + case)
    V = int(rs.integers(1, 400))
    x = (rs.normal(size=V) * rs.choice([0.3, 1.0, 4.0])).astype(np.float32)
    if case % 5 == 0:
        x = np.round(x * 2) / 2  # ties
    T = float(rs.choice([0.0, 0.3, 0.7, 1.0, 2.5]))
    k = int(rs.choice([0, 1, 3, 40, V, V + 5]))
    p = float(rs.choice([1.0, 0.95, 0.5, 0.0]))
    mp = float(rs.choice([0.0, 0.05, 0.3, 2.0]))
    rp = float(rs.choice([1.0, 1.15, 0.8]))
    recent = rs.integers(0, V + 3, size=int(rs.integers(0, 50))).tolist()
    allowed = None
    if case % 7 == 0:
        allowed = (rs.random(V) > 0.3).astype(np.uint8)
    seed = int(rs.integers(0, 1 << 63))
    want, _ = py_sample_with(x, T, k, p, mp, rp, recent, PyRng(seed), allowed=allowed)
    got, _ = one(x, T=T, k=k, p=p, mp=mp, rp=rp, recent=recent, seed=seed, allowed=allowed)
    assert got == want


def test_oracle_probs_match_pure_python():
    rs = np.random.default_rng(5)
    for _ in range(20):
        V = 200
        x = rs.normal(size=V).astype(np.float32) * 2
        seed = int(rs.integers(1 << 60))
        _, kept = py_sample_with(x, 0.8, 40, 0.9, 0.02, 1.0, [], PyRng(seed))
        r = oracle.sample_batch(x[None, :], make_params(0.8, 40, 0.9, 0.02, 1.0),
                                np.array([seed], dtype=np.uint64), want_probs=True)
        assert int(r.kept[0]) == len(kept)
        for i, pv in kept.items():
            assert r.probs[0, i] == np.float32(pv)
        assert np.count_nonzero(r.probs[0]) == len(kept)


def test_batch_threads_agree_with_single_thread():
    from scriptonait_amd.workloads import make_workload

    w = make_workload(2, B=32)
    a = oracle.sample_batch(w.logits, w.params, w.rng_seeds, w.hist, w.hist_offsets, V=w.V, threads=1)
    b = oracle.sample_batch(w.logits, w.params, w.rng_seeds, w.hist, w.hist_offsets, V=w.V, threads=8)
    assert np.array_equal(a.ids, b.ids) and np.array_equal(a.rng_state, b.rng_state)


def test_per_row_params_match_shared():
    from scriptonait_amd.workloads import make_workload

    w = make_workload(1)
    per = np.repeat(w.params, w.B).astype(PARAMS_DTYPE)
    a = oracle.sample_batch(w.logits, w.params, w.rng_seeds, w.hist, w.hist_offsets, V=w.V)
    b = oracle.sample_batch(w.logits, per, w.rng_seeds, w.hist, w.hist_offsets, V=w.V)
    assert np.array_equal(a.ids, b.ids)


def test_softmax_sum_is_a_left_fold_in_sorted_order():
    """The softmax sum (generate.rs:374) adds the terms one at a time in
    sorted order. Terms [t, t, 1] by id with 2^-25 < t < 2^-24 (t = expf(-17)):
    in sorted order 1 + t rounds back to 1 (t is under half an ulp of 1), twice,
    so S = 1 and p_max = 1 exactly, and the top-p cumulative reaches
    top_p = 1 - 2^-24 at the first term (kept 1). An id-order, ascending or
    pairwise sum adds t + t = 2t first, which is over half an ulp: S = 1 + 2^-23,
    p_max = 1 - 2^-23 < top_p, and two terms are kept. The same holds with a
    thousand small terms, where any order other than the sorted one moves S by
    about 4e-5."""
    t64 = np.exp(-17.0)
    assert 2.0 ** -25 < t64 < 2.0 ** -24
    top_p = np.float32(1.0) - np.float32(2.0 ** -24)
    assert float(top_p) == 1.0 - 2.0 ** -24
    for n_small in (2, 1000):
        x = np.full(n_small + 1, -17.0, dtype=np.float32)
        x[-1] = 0.0  # the maximum has the largest id: id order puts it last
        prm = make_params(1.0, 0, float(top_p), 0.0, 1.0)
        seeds = np.arange(16, dtype=np.uint64)
        r = oracle.sample_batch(np.repeat(x[None, :], 16, axis=0), prm, seeds, want_probs=True)
        assert np.all(r.ids == n_small)
        assert np.all(r.kept == 1)
        assert np.all(r.probs[:, -1] == np.float32(1.0))
        assert np.all(r.probs[:, :-1] == 0.0)  # truncated by top-p: not among the kept terms
