"""The reference's sampler tests (crates/llm-core/src/generate.rs:550-692),
run through the drop-in API (scriptonait_amd.sampler: SamplingConfig, Rng,
sample_with, sample), so every sample here is computed by the HIP kernels."""
import numpy as np
import pytest

from scriptonait_amd.sampler import Rng, SamplingConfig, sample, sample_with

pytestmark = pytest.mark.gpu


def test_top_k_restricts_the_choice_to_the_k_best():
    logits = [0.0, 5.0, 0.0, 9.0, 0.0]
    cfg = SamplingConfig(temperature=5.0, top_k=2, top_p=1.0, repetition_penalty=1.0)
    for seed in range(50):
        picked = sample_with(logits, cfg, [], Rng.seed_from_u64(seed))
        assert picked in (3, 1), f"top_k leaked token {picked}"


def test_top_p_keeps_the_nucleus():
    logits = [20.0, 0.0, 0.0, 0.0]
    cfg = SamplingConfig(temperature=1.0, top_k=0, top_p=0.9, repetition_penalty=1.0)
    for seed in range(20):
        assert sample_with(logits, cfg, [], Rng.seed_from_u64(seed)) == 0


def test_repetition_penalty_pushes_recent_tokens_down():
    logits = [2.0, 1.9, 0.0]
    greedy = SamplingConfig(temperature=0.0, repetition_penalty=1.5)
    rng = Rng.seed_from_u64(1)
    assert sample_with(logits, greedy, [], rng) == 0
    assert sample_with(logits, greedy, [0], rng) == 1


def test_min_p_cuts_the_tail_of_a_confident_step():
    logits = [6.0] + [0.0] * 7
    cfg = SamplingConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=0.1, repetition_penalty=1.0)
    rng = Rng.seed_from_u64(1)
    for _ in range(64):
        assert sample_with(logits, cfg, [], rng) == 0


def test_min_p_keeps_the_field_when_the_model_is_unsure():
    logits = [0.10, 0.05, 0.0, -0.05, -0.10]
    cfg = SamplingConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=0.1, repetition_penalty=1.0)
    rng = Rng.seed_from_u64(2)
    seen = [False] * 5
    for _ in range(500):
        seen[sample_with(logits, cfg, [], rng)] = True
    assert all(seen), f"every token should still be reachable: {seen}"


def test_min_p_always_leaves_a_candidate():
    cfg = SamplingConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=5.0, repetition_penalty=1.0)
    assert sample_with([1.0, 0.9, 0.8], cfg, [], Rng.seed_from_u64(3)) == 0


def test_min_p_is_off_unless_asked_for():
    assert SamplingConfig().min_p == 0.0


def test_rng_advances_like_the_reference():
    """One SplitMix64 step per drawn token, none for greedy (rng.rs:16-34)."""
    from pyref import PyRng

    cfg = SamplingConfig(temperature=0.9, top_k=40, top_p=0.95)
    rng, ref = Rng.seed_from_u64(123), PyRng(123)
    rs = np.random.default_rng(0)
    for _ in range(20):
        x = rs.normal(size=300).astype(np.float32)
        sample_with(x, cfg, [], rng)
        ref.next_u64()
        assert rng.state == ref.state
    sample_with(x, SamplingConfig(temperature=0.0), [], rng)
    assert rng.state == ref.state


def test_plain_sample_wrapper():
    """generate.rs:423-433: temperature only."""
    from oracle import oracle
    from scriptonait_amd.workloads import make_params

    rs = np.random.default_rng(9)
    for seed in range(10):
        x = rs.normal(size=1000).astype(np.float32)
        got = sample(x, 0.8, Rng.seed_from_u64(seed))
        r = oracle.sample_batch(x[None, :], make_params(0.8, 0, 1.0, 0.0, 1.0),
                                np.array([seed], dtype=np.uint64))
        assert got == int(r.ids[0])


def test_generation_loop_with_windowed_history():
    """A decode loop as Generator::step runs it (generate.rs:157-182):
    history = last 128 tokens, one RNG per generation, same ids as the CPU
    sampler on the same logits sequence."""
    from pyref import PyRng, sample_with as py_sample_with

    cfg = SamplingConfig(temperature=0.9, top_k=40, top_p=0.95, min_p=0.05,
                         repetition_penalty=1.1, repetition_window=128, seed=77)
    rs = np.random.default_rng(3)
    V = 512
    tokens = list(rs.integers(0, V, size=20))
    rng, ref = Rng.seed_from_u64(cfg.seed), PyRng(cfg.seed)
    for _ in range(60):
        x = (rs.normal(size=V) * 2).astype(np.float32)
        recent = tokens[-cfg.repetition_window:]
        got = sample_with(x, cfg, recent, rng)
        want, _ = py_sample_with(x, cfg.temperature, cfg.top_k, cfg.top_p, cfg.min_p,
                                 cfg.repetition_penalty, recent, ref)
        assert got == want
        tokens.append(got)
