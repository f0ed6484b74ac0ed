"""The synthetic benchmark inputs are deterministic and have the stated shapes
and distributions."""
import numpy as np
import pytest

from scriptonait_amd.workloads import CONFIGS, make_workload, splitmix64_outputs


@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_deterministic(cfg):
    a = make_workload(cfg, B=4)
    b = make_workload(cfg, B=4)
    assert np.array_equal(a.logits, b.logits)
    assert np.array_equal(a.rng_seeds, b.rng_seeds)
    if a.hist is not None:
        assert np.array_equal(a.hist, b.hist)


def test_shapes_and_bytes_per_row():
    w = make_workload(4, B=3)
    assert w.logits.shape == (3, 50260) and w.V == 50257 and w.ld == 50260
    assert w.hist is None and w.bytes_per_row() == 4 * 50257 + 20
    w = make_workload(3, B=2)
    assert w.bytes_per_row() == 132116
    assert make_workload(1).bytes_per_row() == 33812
    assert make_workload(2, B=1).bytes_per_row() == 34836


def test_distributions():
    w = make_workload(3, B=4)
    assert abs(w.logits[0].std() - 0.5) < 0.02 and abs(w.logits[1].std() - 4.0) < 0.1
    w = make_workload(2, B=2)
    # one +12 spike per row on N(0, 3^2)
    from scriptonait_amd.workloads import DEFAULT_DATA_SEED, _substream, normal

    base = (3.0 * normal(_substream(DEFAULT_DATA_SEED, 1000003 * 1 + 2), w.V)).astype(np.float32)
    d = w.logits[0] - base
    assert np.count_nonzero(np.abs(d) > 1e-3) == 1 and abs(d.max() - 12.0) < 1e-3
    h = w.hist[:512]
    assert np.unique(h).size < 512  # Zipf histories repeat ids
    w = make_workload(5, B=1, V=4096)
    assert abs(w.logits[0].mean() - (0.5772 + 0.01)) < 0.1  # Gumbel mean + tilt


def test_histories_in_range():
    for cfg in (1, 2, 3):
        w = make_workload(cfg, B=2)
        assert w.hist.max() < w.V and w.hist_offsets[-1] == w.hist.size


def test_splitmix_stream_offsets():
    a = splitmix64_outputs(5, 10)
    b = splitmix64_outputs(5, 4, start=6)
    assert np.array_equal(a[6:], b)


def test_config_table_matches_baseline():
    assert CONFIGS[3]["B"] == 256 and CONFIGS[3]["V"] == 32000 and CONFIGS[3]["k"] == 64
    assert CONFIGS[5]["V"] == 131072 and CONFIGS[5]["H"] == 2048


def test_prompt_ring_tokens_follow_generator_new():
    """generate.rs:131-139: an empty prompt is [BOS]; a long prompt keeps its
    last context_len tokens; others are unchanged."""
    from scriptonait_amd.sampler import BOS, prompt_ring_tokens

    assert prompt_ring_tokens([], 8).tolist() == [BOS]
    assert prompt_ring_tokens([5, 6, 7], 8).tolist() == [5, 6, 7]
    assert prompt_ring_tokens(list(range(10)), 4).tolist() == [6, 7, 8, 9]
    assert prompt_ring_tokens([], 1).tolist() == [BOS]
    assert prompt_ring_tokens([1, 2], 2).tolist() == [1, 2]
