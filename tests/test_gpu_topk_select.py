"""GPU: top-k rows beyond the headline K against the oracle.

Rows with 64 < top_k <= 4096 and V <= 32768 stay in the fast kernel's
large-K variant. With V > 32768 the streaming kernel takes the K its list
holds (top_k * ceil(V / 32768) * 5 <= 16384, penalty >= 1: here V = 40000
with K = 50 or 1100, V = 50257 with K = 50, V = 131072 with K = 64); the
sorting path takes larger K and the rows either kernel hands over: it
selects the K largest keys from a bound (or a radix select) and sorts them
in LDS, and K > 4096 sorts the whole row in HBM scratch. All must give the
reference's order: key descending, ties by ascending id
(crates/llm-core/src/generate.rs:364-367).
"""
import numpy as np
import pytest

from parity_util import compare, run_both
from scriptonait_amd.workloads import make_params, make_workload

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("k", [1025, 2000, 4096, 4097, 20000, 31999])
def test_top_k_above_the_fast_limit(sampler, k):
    w = make_workload(3, B=16)
    prm = make_params(0.7, k, 0.95, 0.0, 1.15)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, f"k={k}")


@pytest.mark.parametrize("V,k", [(32000, 1100), (32000, 3000), (40000, 50), (40000, 1100), (40000, 3000)])
def test_top_k_select_with_ties_at_the_cut(sampler, V, k):
    """Logits on a coarse grid: the K-th key is shared by hundreds of ids, of
    which only the lowest ids are kept (V = 40000: K = 50 and 1100 go to
    the streaming kernel, which lists every id at its threshold or, when
    they overflow its list, hands the row to the sorting path in its own
    workgroup; K = 3000 goes to the sorting path's LDS select, whose waves
    meet their ids in ascending order)."""
    w = make_workload(3, B=16, V=V)
    w.logits[:] = np.round(w.logits * 2.0) / 2.0
    prm = make_params(1.3, k, 1.0, 0.0, 1.0)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, f"quantized V={V} k={k}")


@pytest.mark.parametrize("case", ["long_tie_runs", "crowded_bound"])
def test_sorting_path_select_fallbacks(sampler, case):
    """V = 40000 top-k rows whose bound cannot be used as is: T = 100 makes
    division merge runs of about 200 adjacent keys (longer than the tie
    lowering covers: the streaming kernel hands these K = 50 rows to the
    sorting path in its own workgroup), and logits on a grid of step 6 put
    thousands of ids on the value at the bound (more candidates than the
    list holds). Both divide every key and select exactly; ids, kept counts,
    probabilities and RNG states match the oracle."""
    w = make_workload(3, B=16, V=40000)
    if case == "long_tie_runs":
        prm = make_params(100.0, 50, 0.9, 0.0, 1.0)
    else:
        w.logits[:] = np.round(w.logits / 6.0) * 6.0
        prm = make_params(1.0, 2000, 0.95, 0.0, 1.0)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, case)


def test_top_k_select_fewer_allowed_than_k(sampler):
    """Only 700 ids allowed and K = 2000: the cut falls among the -inf keys."""
    w = make_workload(3, B=8)
    allowed = np.zeros(w.V, dtype=np.uint8)
    allowed[np.random.default_rng(3).choice(w.V, 700, replace=False)] = 1
    prm = make_params(0.9, 2000, 0.9, 0.02, 1.2)
    g, o = run_both(sampler, w, params=prm, allowed=allowed)
    compare(g, o, "700 allowed, k=2000")


@pytest.mark.parametrize("k", [1, 64, 1000])
def test_hand_over_rows_penalty_below_one(sampler, k):
    """A penalty below 1 can raise a value, so the fast kernel hands these
    rows to the sorting path (which selects in LDS)."""
    w = make_workload(3, B=16)
    prm = make_params(0.8, k, 0.95, 0.05, 0.85)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, f"rp<1 k={k}")


@pytest.mark.parametrize("V,k", [(4097, 4096), (5000, 4999), (40000, 3000), (131072, 4000), (50257, 50),
                                 (40000, 2048), (131072, 64)])
def test_top_k_select_other_vocab_sizes(sampler, V, k):
    w = make_workload(3, B=4, V=V)
    prm = make_params(1.0, k, 0.98, 0.01, 1.1)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, f"V={V} k={k}")


@pytest.mark.parametrize("k", [1025, 2000, 3000, 4096])
@pytest.mark.parametrize("filters", [(0.7, 0.95, 0.05, 1.15), (1.0, 1.0, 0.0, 1.0), (0.9, 0.9, 0.0, 1.3)])
def test_register_path_k_above_1024(sampler, k, filters):
    """1024 < K <= 4096 stays in the fast kernel: the threshold is narrowed
    per slot to the K-th largest known value, the candidates are listed over
    the scan entries' LDS and merge-sorted there, and the tail's terms are
    staged by every wave. Ids, kept counts, probabilities and RNG states
    match the oracle, and no row is handed to the sorting path."""
    T, top_p, min_p, rp = filters
    w = make_workload(3, B=32)
    prm = make_params(T, k, top_p, min_p, rp)
    sampler.status()  # clears the hand-over count
    g, o = run_both(sampler, w, params=prm)
    assert sampler.status().handovers == 0
    compare(g, o, f"k={k} filters={filters}")


@pytest.mark.parametrize("V,k", [(12000, 3000), (8000, 2500), (12001, 2000), (16384, 4096)])
def test_register_path_k_above_1024_other_vocab_sizes(sampler, V, k):
    """1024 < K <= 4096 with four or two chunks per lane (V = 12000, 8000:
    fewer chunk maxima than K, so every known value is counted), an
    unaligned row (V = 12001: scalar loads), and K = 4096 at V = 16384.
    Rows the register path cannot bound may be handed over; every row must
    match the oracle."""
    w = make_workload(3, B=16, V=V)
    prm = make_params(0.8, k, 0.95, 0.0, 1.15)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, f"V={V} k={k}")


@pytest.mark.parametrize("k", [350, 512, 2000])
def test_register_path_retries_with_a_mask_and_penalty(sampler, k):
    """K = 350 / 512 take the proven threshold (the speculative one is not
    used past K = 384, or undercut) and K = 2000 the per-slot narrowing, here
    with a mask that disallows a tenth of the ids and a penalty of 1.3 over
    the history: masked and penalized slots are not known values, so the
    threshold must come from the others. Every row matches the oracle and
    none is handed to the sorting path."""
    w = make_workload(3, B=32)
    allowed = (np.random.default_rng(k).random(w.V) >= 0.1).astype(np.uint8)
    prm = make_params(0.8, k, 0.97, 0.01, 1.3)
    sampler.status()  # clears the hand-over count
    g, o = run_both(sampler, w, params=prm, allowed=allowed)
    assert sampler.status().handovers == 0
    compare(g, o, f"k={k} masked, rp=1.3")


@pytest.mark.parametrize("k", [65, 128, 700, 1024])
@pytest.mark.parametrize("filters", [(0.7, 0.95, 0.05, 1.15), (1.0, 1.0, 0.0, 1.0)])
def test_fast_kernel_k_above_64(sampler, k, filters):
    """64 < K <= 1024 stays in the fast kernel; its tail folds the terms from LDS."""
    T, top_p, min_p, rp = filters
    w = make_workload(3, B=32)
    prm = make_params(T, k, top_p, min_p, rp)
    g, o = run_both(sampler, w, params=prm)
    compare(g, o, f"k={k} filters={filters}")


@pytest.mark.parametrize("K", [128, 2000, 6000])
def test_exact_ties_in_the_lds_tail_folds(sampler, K):
    """128 equal top values give p_i = 1/128 and exact cumulative sums: top-p
    cuts and draws that land exactly on a fold value, decided by the exact
    f32 folds of the LDS tail (generate.rs:397-419); K = 6000 folds over two
    LDS windows."""
    from oracle import oracle
    from scriptonait_amd.workloads import PARAMS_DTYPE
    from test_gpu_parity import _seed_for_draw

    rs = np.random.default_rng(11)
    B, V = 64, 32000
    logits = (rs.standard_normal((B, V)) - 20.0).astype(np.float32)
    for b in range(B):
        logits[b, rs.choice(V, 128, replace=False)] = 5.0
    prm = np.zeros(B, dtype=PARAMS_DTYPE)
    seeds = np.zeros(B, dtype=np.uint64)
    for b in range(B):
        top_p = [0.5, 0.25, 1.0, 0.75 + 2.0 ** -20][b % 4]
        prm[b] = (1.0, K, top_p, [0.0, 0.5][b % 2], 1.0)
        seeds[b] = _seed_for_draw((b % 32) << 19)  # u = (b % 32) / 32
    g = sampler.sample_host(logits, prm, seeds, want_probs=True)
    o = oracle.sample_batch(logits, prm, seeds, want_probs=True)
    assert np.array_equal(g.ids, o.ids), np.nonzero(g.ids != o.ids)[0]
    assert np.array_equal(g.kept, o.kept)
    assert np.array_equal(g.rng_state, o.rng_state)
    assert np.array_equal(g.probs, o.probs)


@pytest.mark.parametrize("k", [2, 9, 40, 64])
def test_register_tail_sum_is_the_reference_fold(sampler, k):
    """K <= 64: the register tail's softmax sum, bit for bit (every
    probability is e_i / sum, all K kept with top_p = 1 and min_p = 0), at
    temperatures that put the sum in one binade or across several."""
    w = make_workload(3, B=32)
    for T in (0.05, 0.7, 1.0, 3.0, 30.0):
        prm = make_params(T, k, 1.0, 0.0, 1.15)
        g, o = run_both(sampler, w, params=prm)
        assert np.array_equal(g.ids, o.ids)
        assert np.array_equal(g.kept, o.kept)
        assert np.array_equal(g.probs.view(np.uint32), o.probs.view(np.uint32)), f"k={k} T={T}"


@pytest.mark.parametrize("k", [65, 300, 700, 1024, 2000, 4096])
def test_lds_tail_sum_is_the_reference_fold(sampler, k):
    """The LDS tail folds the softmax sum term by term in f32, in sorted
    order. Every probability is e_i / sum, so with top_p = 1 and min_p = 0
    (all K kept) the probabilities must equal the oracle's bit for bit, not
    just within the tolerance: one ulp off in the sum would show in every
    one of them."""
    w = make_workload(3, B=24)
    for T in (0.7, 1.0, 3.0):
        prm = make_params(T, k, 1.0, 0.0, 1.15)
        g, o = run_both(sampler, w, params=prm)
        assert np.array_equal(g.ids, o.ids)
        assert np.array_equal(g.kept, o.kept)
        assert np.array_equal(g.probs.view(np.uint32), o.probs.view(np.uint32)), f"k={k} T={T}"
