"""GPU: llmhip_decode_step against a CPU decode loop over the oracle.

The loop is Generator::step (crates/llm-core/src/generate.rs:157-165) with
recent_tokens (generate.rs:178-182): each step samples every live row with
the last `window` tokens of its history (prompt included) as `recent`,
appends the token, and ends the row at EOS. On the device the histories,
lengths, done flags and RNG states stay in HBM across steps; on the CPU the
same loop runs over Python lists with oracle.sample_batch. Every step's ids
and the final rings, lengths, done flags and RNG states must match.

With a context length, the CPU loop also resets each row's cache as
Generator::advance does (maybe_reset_cache, generate.rs:187-196: at
context_len tokens the cache keeps its last context_len / 2 before the new
token is appended), so `recent` is the last window tokens of the cache, not
of the whole history; the device loop is told where each row's cache starts
through hist_start, as a caller would after resetting its model's cache.
"""
import numpy as np
import pytest

from scriptonait_amd.workloads import EOS_ID, make_params

pytestmark = pytest.mark.gpu


def _run(sampler, V, prm, steps=24, B=16, window=128, cap=256, seed=3, context_len=None, max_prompt=300,
         eos_rows=1, counts=False, fixed=0.0):
    import torch

    from oracle import oracle

    rs = np.random.default_rng(seed)
    dev = torch.device("cuda:0")
    prompts = [rs.integers(0, V, size=int(rs.integers(1, max_prompt))).astype(np.uint32) for _ in range(B)]
    ring = np.zeros((B, cap), dtype=np.uint32)
    for b, pr in enumerate(prompts):
        for j, tok in enumerate(pr):
            ring[b, j % cap] = tok
    lens = np.array([len(p) for p in prompts], dtype=np.uint32)
    rng0 = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    d_ring = torch.from_numpy(ring.view(np.int32)).to(dev)
    d_len = torch.from_numpy(lens.view(np.int32)).to(dev)
    d_done = torch.zeros(B, dtype=torch.int32, device=dev)
    d_rng = torch.from_numpy(rng0.view(np.int64)).to(dev)
    d_ids = torch.zeros(B, dtype=torch.int32, device=dev)
    hist = [list(p) for p in prompts]
    cache = [list(p) for p in prompts]  # the model cache's tokens (recent_tokens reads these)
    d_start = torch.zeros(B, dtype=torch.int32, device=dev) if context_len else None
    d_counts = d_counted = None
    if counts:  # the table starts as garbage: a zero counted range makes the first step rebuild it
        d_counts = torch.from_numpy(rs.integers(0, 2**31, size=(B, (V + 1) // 2)).astype(np.int32)).to(dev)
        d_counted = torch.zeros((B, 2), dtype=torch.int32, device=dev)
    resets = 0
    done = np.zeros(B, dtype=bool)
    st = rng0.copy()
    # fixed > 0: every step's logits are one fixed row plus `fixed` times fresh
    # noise, so the generation draws the same top ids again and again and
    # the window fills with the row's own best candidates (the penalty then
    # pushes them below the register path's speculative threshold).
    base = rs.standard_normal((B, V)) * 3.0 if fixed else None
    for t in range(steps):
        if fixed:
            logits = (base + fixed * rs.standard_normal((B, V))).astype(np.float32)
        else:
            logits = (rs.standard_normal((B, V)) * 3.0).astype(np.float32)
        for b in range(0, B, eos_rows):  # some rows end at EOS along the way
            if (b + 3 * t) % 29 == 0:
                logits[b, EOS_ID] = 60.0
        sampler.decode_step(torch.from_numpy(logits).to(dev), prm, d_ring, d_len, d_done, window, d_rng, d_ids,
                            hist_start=d_start, counts=d_counts, counted=d_counted)
        live = np.nonzero(~done)[0]
        want = np.full(B, EOS_ID, dtype=np.uint32)
        if live.size:
            recent = [np.array(cache[b][-window:], dtype=np.uint32) for b in live]
            offs = np.concatenate([[0], np.cumsum([r.size for r in recent])]).astype(np.uint32)
            o = oracle.sample_batch(logits[live], prm, st[live], np.concatenate(recent), offs, V=V)
            want[live] = o.ids
            st[live] = o.rng_state
            for i, b in enumerate(live):
                if o.ids[i] == EOS_ID:
                    done[b] = True
                else:
                    if context_len and len(cache[b]) >= context_len:
                        cache[b] = cache[b][-max(context_len // 2, 1):]
                        resets += 1
                    hist[b].append(int(o.ids[i]))
                    cache[b].append(int(o.ids[i]))
        if d_start is not None:
            d_start.copy_(torch.tensor([len(hist[b]) - len(cache[b]) for b in range(B)], dtype=torch.int32))
        got = d_ids.cpu().numpy().view(np.uint32)
        assert np.array_equal(got, want), (t, np.nonzero(got != want)[0])
    assert done.any() and not done.all()
    if context_len:
        assert resets > 0
    assert np.array_equal(d_done.cpu().numpy() != 0, done)
    assert np.array_equal(d_rng.cpu().numpy().view(np.uint64), st)
    glen = d_len.cpu().numpy().view(np.uint32)
    assert np.array_equal(glen, [len(h) for h in hist])
    gring = d_ring.cpu().numpy().view(np.uint32)
    for b in range(B):
        n = len(hist[b])
        for j in range(max(0, n - cap), n):
            assert gring[b, j % cap] == hist[b][j], (b, j)
    if counts:
        # The table holds the window that the last step of each row used:
        # counted = [len - H, len) at that step; its multiplicities are the
        # window's (ids >= V are not counted).
        tab = d_counts.cpu().numpy().view(np.uint32)
        cnt = d_counted.cpu().numpy().view(np.uint32)
        for b in range(B):
            lo, hi = int(cnt[b, 0]), int(cnt[b, 1])
            assert 0 <= lo <= hi <= len(hist[b])
            want = np.zeros(V, dtype=np.int64)
            for tok in hist[b][lo:hi]:
                if tok < V:
                    want[tok] += 1
            got = np.stack([tab[b] & 0xFFFF, tab[b] >> 16], axis=1).reshape(-1)[:V]
            assert np.array_equal(got, want), b
        return resets
    return resets


def test_decode_loop_top_k_path(sampler):
    """Config-3 parameters, V = 32000 (the register path)."""
    _run(sampler, 32000, make_params(0.7, 64, 0.95, 0.05, 1.15))


def test_decode_loop_full_vocab_path(sampler):
    """top_k = 0 (the bucketed exact-fold path), with a strong penalty and a short window."""
    _run(sampler, 2048, make_params(1.0, 0, 0.9, 0.02, 1.8), window=16, cap=16)


def test_decode_loop_cache_resets(sampler):
    """A window (48) longer than what a cache reset keeps (context_len 64 -> 32
    tokens): recent must come from the cache, so hist_start moves at each reset."""
    _run(sampler, 32000, make_params(0.7, 64, 0.95, 0.05, 1.15), steps=40, window=48, cap=64, context_len=64,
         max_prompt=60, eos_rows=2)


def test_decode_loop_cache_resets_full_vocab(sampler):
    _run(sampler, 2048, make_params(1.0, 0, 0.9, 0.02, 1.8), steps=40, window=48, cap=64, context_len=64,
         max_prompt=60, eos_rows=2)


def test_decode_step_rejects_an_empty_vocabulary(sampler):
    import torch

    from scriptonait_amd.sampler import SamplerError

    dev = torch.device("cuda:0")
    z = torch.zeros((4, 1), dtype=torch.float32, device=dev)
    ring = torch.zeros((4, 8), dtype=torch.int32, device=dev)
    ln = torch.zeros(4, dtype=torch.int32, device=dev)
    rng = torch.zeros(4, dtype=torch.int64, device=dev)
    ids = torch.zeros(4, dtype=torch.int32, device=dev)
    with pytest.raises(SamplerError):
        sampler.decode_step(z, make_params(0.7, 64, 0.95, 0.05, 1.15), ring, ln, None, 8, rng, ids, V=0)


def test_decode_loop_greedy(sampler):
    _run(sampler, 8192, make_params(0.0, 64, 0.95, 0.05, 1.3))


@pytest.mark.parametrize("path", ["top_k", "full_vocab", "greedy"])
def test_decode_loop_with_count_table(sampler, path):
    """llmhip_decode_step_counts: the same ids, rings and RNG states as the
    CPU loop, and a count table equal to the window's multiplicities."""
    if path == "top_k":
        _run(sampler, 32000, make_params(0.7, 64, 0.95, 0.05, 1.15), counts=True)
    elif path == "full_vocab":
        _run(sampler, 2048, make_params(1.0, 0, 0.9, 0.02, 1.8), window=16, cap=17, counts=True)
    else:
        _run(sampler, 8192, make_params(0.0, 64, 0.95, 0.05, 1.3), counts=True)


@pytest.mark.parametrize("k", [64, 300, 700, 2000])
@pytest.mark.parametrize("counts", [False, True])
def test_decode_loop_drawing_its_own_top_ids(sampler, k, counts):
    """Logits that barely change from step to step: the window fills with
    the rows' own top candidates, so the register path's retries (a second
    speculative pass, the proven threshold from per-thread or per-chunk
    known maxima) and, with a count table, its table reads for those
    retries run at every step. Ids, rings and RNG states match the CPU loop
    step by step."""
    _run(sampler, 32000, make_params(0.8, k, 0.97, 0.0, 1.3), steps=40, B=16, window=256, cap=320,
         max_prompt=50, counts=counts, fixed=0.3, eos_rows=4)


def test_decode_loop_greedy_drawing_its_own_top_ids(sampler):
    """Greedy rows whose window holds their own argmax again and again: the
    penalty bound (only history slots at or above the largest known value
    are penalized) must still give the reference's argmax."""
    _run(sampler, 32000, make_params(0.0, 64, 0.95, 0.05, 1.05), steps=40, B=16, window=256, cap=320,
         max_prompt=50, fixed=0.3, eos_rows=4)
    _run(sampler, 32000, make_params(0.0, 64, 0.95, 0.05, 1.05), steps=40, B=16, window=256, cap=320,
         max_prompt=50, fixed=0.3, counts=True, eos_rows=4)


@pytest.mark.parametrize("counts", [False, True])
@pytest.mark.parametrize("k", [50, 2000])
def test_decode_loop_large_vocab_top_k(sampler, counts, k):
    """V = 40000 top-k rows (beyond the register path's V) inside a decode
    loop, with the ring's window as the history (and the count table kept
    current): top_k = 50 runs the streaming kernel's decode-step variant,
    top_k = 2000 (more than its list holds at this V) the sorting path's
    select bound, list and merge sort."""
    _run(sampler, 40000, make_params(0.7, k, 0.95, 0.05, 1.15), steps=12, B=8, window=256, cap=320,
         max_prompt=200, counts=counts)


def test_decode_loop_with_count_table_and_cache_resets(sampler):
    """hist_start jumps at each cache reset: the table is rebuilt there and
    slid between resets."""
    resets = _run(sampler, 32000, make_params(0.7, 64, 0.95, 0.05, 1.15), steps=40, window=48, cap=64,
                  context_len=64, max_prompt=60, eos_rows=2, counts=True)
    assert resets > 0


def test_decode_loop_with_a_long_window_count_table(sampler):
    """A 3000-token window (prompts of up to 4000 uniform tokens, so ids repeat):
    the table slides one token a step over a long window."""
    _run(sampler, 32000, make_params(0.7, 64, 0.95, 0.05, 1.15), steps=12, B=8, window=3000, cap=4096,
         max_prompt=4000, counts=True)
