"""GPU: the allowed mask as bits. llmhip_seen_tokens against the oracle's
restatement of Corpus::seen_tokens (crates/llm-core/src/corpus.rs:236-247),
and llmhip_sample_device_bits / llmhip_decode_step_bits against the oracle
(and the byte-mask entries) with that mask as SamplingConfig::allowed
(generate.rs:333-341). Ids, kept counts and RNG states must be equal."""
import numpy as np
import pytest

from oracle import oracle
from scriptonait_amd.workloads import EOS_ID, make_params

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("V,n", [(1, 5), (31, 0), (32, 100), (33, 100), (259, 200000), (8192, 3000),
                                 (50257, 100000), (131072, 2000000), (600000, 50000)])
def test_seen_tokens_bits(sampler, V, n):
    """Repeated ids, ids >= V, V not a multiple of 32, an empty corpus, and a
    mask too large for the kernel's LDS copy (V = 600000)."""
    import torch

    rs = np.random.default_rng(V + n)
    tok = np.concatenate([rs.integers(0, V + 100, size=n // 2),
                          rs.integers(0, min(V, 50), size=n - n // 2)]).astype(np.uint32)
    rs.shuffle(tok)
    dev = torch.device("cuda:0")
    t = torch.from_numpy(tok.view(np.int32)).to(dev)
    out = torch.full(((V + 31) // 32,), -1, dtype=torch.int32, device=dev)  # stale bits must go
    sampler.seen_tokens(t, V, out_bits=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, oracle.pack_bits(oracle.seen_tokens(tok, V)))


def _case(sampler, V, prm, B, allowed_len, seed, with_hist):
    import torch

    rs = np.random.default_rng(seed)
    dev = torch.device("cuda:0")
    logits = (rs.standard_normal((B, V)) * 2.5).astype(np.float32)
    corpus = rs.integers(0, V + 20, size=max(1, allowed_len // 2)).astype(np.uint32)
    seen = oracle.seen_tokens(corpus, allowed_len)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    hist = offs = None
    if with_hist:
        H = 300
        hist = rs.integers(0, V, size=B * H).astype(np.uint32)
        offs = (np.arange(B + 1) * H).astype(np.uint32)
    o = oracle.sample_batch(logits, prm, seeds, hist, offs, allowed=seen.astype(np.uint8), V=V, threads=8)

    d_logits = torch.from_numpy(logits).to(dev)
    d_hist = torch.from_numpy(hist.view(np.int32)).to(dev) if with_hist else None
    d_offs = torch.from_numpy(offs.view(np.int32)).to(dev) if with_hist else None
    d_corpus = torch.from_numpy(corpus.view(np.int32)).to(dev)
    d_bits = sampler.seen_tokens(d_corpus, allowed_len)
    d_bytes = torch.from_numpy(seen.astype(np.uint8)).to(dev)
    got = {}
    for kind in ("bits", "bytes"):
        d_rng = torch.from_numpy(seeds.view(np.int64)).to(dev)
        d_ids = torch.zeros(B, dtype=torch.int32, device=dev)
        d_kept = torch.zeros(B, dtype=torch.int32, device=dev)
        if kind == "bits":
            sampler.sample_device(d_logits, prm, d_rng, d_ids, V=V, hist=d_hist, hist_offsets=d_offs,
                                  allowed_bits=d_bits, allowed_len=allowed_len, out_kept=d_kept)
        else:
            sampler.sample_device(d_logits, prm, d_rng, d_ids, V=V, hist=d_hist, hist_offsets=d_offs,
                                  allowed=d_bytes, out_kept=d_kept)
        torch.cuda.synchronize()
        got[kind] = (d_ids.cpu().numpy().view(np.uint32), d_rng.cpu().numpy().view(np.uint64),
                     d_kept.cpu().numpy().view(np.uint32))
    for kind, (ids, st, kept) in got.items():
        bad = np.nonzero(ids != o.ids)[0]
        assert bad.size == 0, (kind, bad[:8], ids[bad[:8]], o.ids[bad[:8]])
        assert np.array_equal(st, o.rng_state), kind
        assert np.array_equal(kept, o.kept), kind
    assert not seen.all() and seen.any()


def test_bits_on_the_register_path(sampler):
    _case(sampler, 8192, make_params(0.8, 40, 0.95, 0.05, 1.1), B=48, allowed_len=8192, seed=1, with_hist=True)


def test_bits_covering_part_of_the_vocabulary(sampler):
    """Ids >= allowed_len are always allowed."""
    _case(sampler, 8192, make_params(1.0, 50, 0.9, 0.0, 1.0), B=48, allowed_len=5000, seed=2, with_hist=False)


def test_bits_on_the_full_vocabulary_path(sampler):
    _case(sampler, 9000, make_params(0.9, 0, 0.95, 0.02, 1.2), B=32, allowed_len=9000, seed=3, with_hist=True)


def test_bits_on_the_sorting_path(sampler):
    _case(sampler, 5000, make_params(1.1, 2000, 0.9, 0.0, 1.3), B=16, allowed_len=5000, seed=4, with_hist=True)


def test_bits_greedy_rows(sampler):
    _case(sampler, 4096, make_params(0.0, 0, 1.0, 0.0, 1.2), B=16, allowed_len=4096, seed=5, with_hist=True)


def test_decode_step_bits_matches_the_byte_mask(sampler):
    """Eight decode steps with the mask as bits and as bytes: every step's ids
    and the final rings, lengths, done flags and RNG states agree."""
    import torch

    rs = np.random.default_rng(6)
    dev = torch.device("cuda:0")
    B, V, cap, window = 12, 32000, 64, 32
    prm = make_params(0.7, 64, 0.95, 0.05, 1.15)
    corpus = rs.integers(0, V, size=12000).astype(np.uint32)
    corpus = np.append(corpus, np.uint32(EOS_ID))
    seen = oracle.seen_tokens(corpus, V)
    ring0 = rs.integers(0, V, size=(B, cap)).astype(np.uint32)
    len0 = rs.integers(1, cap, size=B).astype(np.uint32)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    d_bits = sampler.seen_tokens(torch.from_numpy(corpus.view(np.int32)).to(dev), V)
    d_bytes = torch.from_numpy(seen.astype(np.uint8)).to(dev)
    state = {}
    for kind in ("bits", "bytes"):
        state[kind] = dict(ring=torch.from_numpy(ring0.view(np.int32)).to(dev),
                           len=torch.from_numpy(len0.view(np.int32)).to(dev),
                           done=torch.zeros(B, dtype=torch.int32, device=dev),
                           rng=torch.from_numpy(seeds.view(np.int64)).to(dev),
                           ids=torch.zeros(B, dtype=torch.int32, device=dev))
    for t in range(8):
        logits = (rs.standard_normal((B, V)) * 3.0).astype(np.float32)
        logits[t % B, EOS_ID] = 50.0
        d_logits = torch.from_numpy(logits).to(dev)
        for kind, s in state.items():
            kw = dict(allowed_bits=d_bits) if kind == "bits" else dict(allowed=d_bytes)
            sampler.decode_step(d_logits, prm, s["ring"], s["len"], s["done"], window, s["rng"], s["ids"], **kw)
        torch.cuda.synchronize()
        a, b = state["bits"]["ids"].cpu().numpy(), state["bytes"]["ids"].cpu().numpy()
        assert np.array_equal(a, b), t
        assert all(seen[i] or i == EOS_ID for i in a.view(np.uint32))
    for key in ("ring", "len", "done", "rng"):
        assert torch.equal(state["bits"][key], state["bytes"][key]), key
    assert state["bits"]["done"].any()
