"""GPU: llmhip_sample_device_noalloc against llmhip_sample_device.

The no-alloc entry runs the same kernels as llmhip_sample_device, with its
device memory (per-row parameters, the allowed mask's slot layout, the
sorting path's per-row scratch) taken from the library's fixed per-GPU array
instead of the context's buffers. Three calls in a row, each smaller than
the last and of another kind, must give the same ids, RNG states, kept counts and
probabilities as llmhip_sample_device on the same inputs: the array keeps the
first call's contents, so the later ones show that nothing depends on what
an earlier call left there. A call larger than the array is refused with
LLMHIP_ERR_UNSUPPORTED before anything is enqueued.
"""
import numpy as np
import pytest

from scriptonait_amd import sampler as smp
from scriptonait_amd.workloads import make_workload

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 96 << 20  # LLMHIP_NOALLOC_SCRATCH_BYTES


def _both_entries(sampler, w, params, allowed=None, want_probs=False):
    """Run llmhip_sample_device and llmhip_sample_device_noalloc on the same
    device inputs; returns both results as numpy arrays."""
    import torch

    dev = torch.device("cuda:0")
    lg = torch.from_numpy(np.ascontiguousarray(w.logits)).to(dev)
    hs = offs = None
    if w.hist is not None:
        hs = torch.from_numpy(w.hist.view(np.int32)).to(dev)
        offs = torch.from_numpy(w.hist_offsets.view(np.int32)).to(dev)
    al = None if allowed is None else torch.from_numpy(allowed).to(dev)
    out = []
    for noalloc in (False, True):
        rng = torch.from_numpy(w.rng_seeds.view(np.int64).copy()).to(dev)
        ids = torch.full((w.B,), -1, dtype=torch.int32, device=dev)
        kept = torch.full((w.B,), -1, dtype=torch.int32, device=dev)
        probs = torch.full((w.B, w.V), -1.0, dtype=torch.float32, device=dev) if want_probs else None
        sampler.sample_device(lg, params, rng, ids, V=w.V, hist=hs, hist_offsets=offs, allowed=al,
                              out_probs=probs, out_kept=kept, noalloc=noalloc)
        torch.cuda.synchronize()
        out.append(dict(ids=ids.cpu().numpy().view(np.uint32), rng=rng.cpu().numpy().view(np.uint64),
                        kept=kept.cpu().numpy().view(np.uint32),
                        probs=None if probs is None else probs.cpu().numpy()))
    return out


def _same(a, b):
    assert np.array_equal(a["ids"], b["ids"])
    assert np.array_equal(a["rng"], b["rng"])
    assert np.array_equal(a["kept"], b["kept"])
    if a["probs"] is not None:
        assert np.array_equal(a["probs"].view(np.uint32), b["probs"].view(np.uint32))


def test_noalloc_matches_the_allocating_entry_twice_in_a_row(sampler):
    from oracle import oracle

    print("no-alloc call 1: config 3, B=256, V=32000, per-row params, rp < 1 on some rows", flush=True)
    w = make_workload(3)
    prm = np.repeat(w.params, w.B)
    prm["repetition_penalty"][np.arange(w.B) % 16 == 5] = 0.85  # handed to the sorting path (scratch)
    prm["top_k"][np.arange(w.B) % 16 == 9] = 2000  # the register path's large-K kernel (no scratch)
    sampler.status()
    first = _both_entries(sampler, w, prm)
    _same(*first)
    st = sampler.status()
    assert st.flags == 0
    assert st.handovers == 2 * int((np.arange(w.B) % 16 == 5).sum())  # once per entry
    o = oracle.sample_batch(w.logits, prm, w.rng_seeds, w.hist, w.hist_offsets, V=w.V)
    assert np.array_equal(first[1]["ids"], o.ids)

    print("no-alloc call 2: config 4 shape, B=24, V=50257, allowed mask, probabilities", flush=True)
    w2 = make_workload(4, B=24)
    prm2 = np.repeat(w2.params, w2.B)
    prm2["top_k"][1::3] = 4500  # whole-row sort (5 scratch words per row)
    prm2["temperature"][2::5] = 0.0  # greedy
    allowed = (np.arange(w2.V) % 7 != 3).astype(np.uint8)
    second = _both_entries(sampler, w2, prm2, allowed=allowed, want_probs=True)
    _same(*second)
    assert sampler.status().flags == 0
    o2 = oracle.sample_batch(w2.logits, prm2, w2.rng_seeds, None, None, V=w2.V, allowed=allowed,
                             want_probs=True)
    assert np.array_equal(second[1]["ids"], o2.ids)
    assert np.array_equal(second[1]["rng"], o2.rng_state)

    print("no-alloc call 3: B=12, V=50257, top_k 40 (streaming kernel) and 2000 (the sorting path's select, "
          "keys in the array)", flush=True)
    w3 = make_workload(4, B=12)
    prm3 = np.repeat(w3.params, w3.B)
    # K = 2000 at V = 50257 is past what the streaming kernel's list holds, so
    # those rows take the sorting path, whose keys live in the array.
    prm3["top_k"] = np.where(np.arange(w3.B) % 2 == 0, 40, 2000)
    prm3["repetition_penalty"] = 1.1
    rs = np.random.default_rng(3)
    w3.hist = rs.integers(0, w3.V, size=w3.B * 300).astype(np.uint32)
    w3.hist_offsets = (np.arange(w3.B + 1) * 300).astype(np.uint32)
    third = _both_entries(sampler, w3, prm3)
    _same(*third)
    assert sampler.status().flags == 0
    o3 = oracle.sample_batch(w3.logits, prm3, w3.rng_seeds, w3.hist, w3.hist_offsets, V=w3.V)
    assert np.array_equal(third[1]["ids"], o3.ids)
    assert np.array_equal(third[1]["rng"], o3.rng_state)


def test_noalloc_refuses_a_call_beyond_its_array(sampler):
    import torch

    dev = torch.device("cuda:0")
    B, V = 256, 131072  # top_k = 0: 5 scratch words per id and row, 640 MiB > 96 MiB
    lg = torch.zeros((B, V), dtype=torch.float32, device=dev)
    rng = torch.zeros(B, dtype=torch.int64, device=dev)
    ids = torch.full((B,), -7, dtype=torch.int32, device=dev)
    prm = np.zeros(1, dtype=smp.PARAMS_DTYPE)
    prm["temperature"] = 1.0
    prm["top_p"] = 1.0
    prm["repetition_penalty"] = 1.0
    with pytest.raises(smp.SamplerError) as ei:
        sampler.sample_device(lg, prm, rng, ids, V=V, noalloc=True)
    assert ei.value.status == -5
    assert str(NOALLOC_BYTES) in str(ei.value)
    torch.cuda.synchronize()
    assert (ids.cpu().numpy() == -7).all()  # nothing was enqueued
