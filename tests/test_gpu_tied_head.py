"""GPU: llmhip_sample_tied_head_device against the oracle.

The reference's decode step computes logits = final_normed @ embed^T with
ops::linear_fwd (crates/llm-core/src/model.rs:396-397, ops/linear.rs:
19-32, 110-125) and samples them with sample_with. The GPU entry must give
the same logits bit for bit (compared with ==, where -0.0 == +0.0: the sign
of a zero logit changes nothing downstream) and the same ids, kept counts
and RNG states as the oracle's linear_fwd followed by its sample_with.
"""
import numpy as np
import pytest

from oracle import oracle
from scriptonait_amd.workloads import make_params

pytestmark = pytest.mark.gpu


def _case(rs, B, V, h, scale=0.02):
    hidden = rs.standard_normal((B, h)).astype(np.float32)
    embed = (scale * rs.standard_normal((V, h))).astype(np.float32)
    return hidden, embed


def _run(sampler, hidden, embed, prm, seeds, hist=None, offs=None, take_logits=True, ldh=None):
    import torch

    dev = torch.device("cuda:0")
    B, h = hidden.shape
    V = embed.shape[0]
    if ldh is not None:  # rows at a stride that is not a multiple of 4 floats
        padded = np.zeros((B, ldh), dtype=np.float32)
        padded[:, :h] = hidden
        d_hidden = torch.from_numpy(padded).to(dev)[:, :h]
    else:
        d_hidden = torch.from_numpy(hidden).to(dev)
    d_embed = torch.from_numpy(embed).to(dev)
    rng = torch.from_numpy(seeds.view(np.int64).copy()).to(dev)
    ids = torch.zeros(B, dtype=torch.int32, device=dev)
    kept = torch.zeros(B, dtype=torch.int32, device=dev)
    lg = torch.full((B, V), float("nan"), dtype=torch.float32, device=dev) if take_logits else None
    hs = os_ = None
    if hist is not None:
        hs = torch.from_numpy(hist.view(np.int32)).to(dev)
        os_ = torch.from_numpy(offs.view(np.int32)).to(dev)
    sampler.sample_tied_head_device(d_hidden, d_embed, prm, rng, ids, hist=hs, hist_offsets=os_, out_kept=kept,
                                    out_logits=lg)
    torch.cuda.synchronize()
    return (ids.cpu().numpy().view(np.uint32), rng.cpu().numpy().view(np.uint64), kept.cpu().numpy().view(np.uint32),
            None if lg is None else lg.cpu().numpy())


def _check(got, hidden, embed, prm, seeds, hist=None, offs=None):
    ids, rng, kept, lg = got
    want_lg = oracle.linear_fwd(hidden, embed, threads=8)
    if lg is not None:
        bad = np.nonzero(~(lg == want_lg))
        assert bad[0].size == 0, f"logits differ at {list(zip(*bad))[:5]}"
    o = oracle.sample_batch(want_lg, prm, seeds, hist, offs, V=embed.shape[0], threads=8)
    assert np.array_equal(ids, o.ids)
    assert np.array_equal(rng, o.rng_state)
    assert np.array_equal(kept, o.kept)


@pytest.mark.parametrize("h", [256, 512])
def test_config3_shape(sampler, h):
    """V = 32000, B = 64, config 3's filters and a 1024-token history."""
    rs = np.random.default_rng(h)
    B, V = 64, 32000
    hidden, embed = _case(rs, B, V, h)
    H = 1024
    hist = rs.integers(0, V, size=B * H).astype(np.uint32)
    offs = (np.arange(B + 1) * H).astype(np.uint32)
    prm = make_params(0.7, 64, 0.95, 0.05, 1.15)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    got = _run(sampler, hidden, embed, prm, seeds, hist, offs)
    _check(got, hidden, embed, prm, seeds, hist, offs)


@pytest.mark.parametrize("B,V,h", [(45, 1000, 257), (3, 130, 5), (33, 4099, 64), (1, 8192, 3)])
def test_ragged_shapes(sampler, B, V, h):
    """B and V off the tile sizes, h off the chunk sizes (the remainder
    fold), tiny h."""
    rs = np.random.default_rng(B * 7 + h)
    hidden, embed = _case(rs, B, V, h, scale=0.5)
    prm = make_params(0.9, 40, 0.9, 0.02, 1.0)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    _check(_run(sampler, hidden, embed, prm, seeds), hidden, embed, prm, seeds)


def test_unaligned_rows_and_context_logits(sampler):
    """Hidden rows 257 floats apart (no 16-byte loads), and the same call
    with the logits kept in the context: the same ids."""
    rs = np.random.default_rng(11)
    B, V, h = 40, 5000, 256
    hidden, embed = _case(rs, B, V, h, scale=0.1)
    prm = make_params(1.0, 50, 0.9, 0.1, 1.0)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    got = _run(sampler, hidden, embed, prm, seeds, ldh=257)
    _check(got, hidden, embed, prm, seeds)
    ids2, rng2, _, _ = _run(sampler, hidden, embed, prm, seeds, take_logits=False)
    assert np.array_equal(ids2, got[0]) and np.array_equal(rng2, got[1])


def test_full_vocabulary_rows(sampler):
    """top_k = 0: the head feeds the full-vocabulary kernel."""
    rs = np.random.default_rng(12)
    B, V, h = 24, 50257, 128
    hidden, embed = _case(rs, B, V, h, scale=0.15)
    prm = make_params(1.0, 0, 0.98, 0.0, 1.0)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    _check(_run(sampler, hidden, embed, prm, seeds, take_logits=False), hidden, embed, prm, seeds)


def test_one_hot_hidden_rows_select_embedding_columns(sampler):
    """hidden = e_j: every logit is embed[o][j] exactly, so greedy picks the
    argmax of column j."""
    rs = np.random.default_rng(13)
    B, V, h = 16, 3000, 64
    embed = rs.standard_normal((V, h)).astype(np.float32)
    hidden = np.zeros((B, h), dtype=np.float32)
    cols = rs.integers(0, h, size=B)
    hidden[np.arange(B), cols] = 1.0
    prm = make_params(0.0, 64, 0.95, 0.05, 1.0)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    ids, _, _, lg = _run(sampler, hidden, embed, prm, seeds)
    assert np.array_equal(lg, embed[:, cols].T)
    assert np.array_equal(ids, np.argmax(embed[:, cols], axis=0).astype(np.uint32))
