"""GPU: llmhip_ctx_status and the test hooks of llmhip_ctx_debug.

The device entries return once their kernels are enqueued, so a kernel that
hits an internal limit (a wait between wavefronts that runs out of spins)
sets a device word instead of a return status. These tests force that
condition from the host: either the word is set directly, or the waits'
spin bound is lowered to one spin, so waits run out while every kernel
still finishes normally. They also check the hand-over count, which says
how many rows a kernel passed to the sorting path.
"""
import numpy as np
import pytest

from scriptonait_amd import sampler as smp
from scriptonait_amd.workloads import make_params, make_workload

pytestmark = pytest.mark.gpu


def _device_call(sampler, w, params=None):
    import torch

    dev = torch.device("cuda:0")
    lg = torch.from_numpy(w.logits).to(dev)
    rng = torch.from_numpy(w.rng_seeds.view(np.int64)).to(dev)
    ids = torch.zeros(w.B, dtype=torch.int32, device=dev)
    hs = offs = None
    if w.hist is not None:
        hs = torch.from_numpy(w.hist.view(np.int32)).to(dev)
        offs = torch.from_numpy(w.hist_offsets.view(np.int32)).to(dev)
    sampler.sample_device(lg, w.params if params is None else params, rng, ids, V=w.V, hist=hs, hist_offsets=offs)
    return ids


def test_clean_call_reports_nothing(sampler):
    sampler.status()  # whatever earlier tests left
    ids = _device_call(sampler, make_workload(3, B=64))
    st = sampler.status()
    assert st.flags == 0 and st.handovers == 0
    assert ids.cpu().numpy().size == 64


def test_handover_count_is_the_rows_passed_to_the_sorting_path(sampler):
    """A penalty below 1 can raise a value past the register path's
    threshold, so the fast kernel hands exactly those rows over."""
    from oracle import oracle

    w = make_workload(3, B=32)
    prm = np.repeat(w.params, w.B)
    below = np.arange(w.B) % 4 == 1
    prm["repetition_penalty"][below] = 0.8
    sampler.status()
    ids = _device_call(sampler, w, prm)
    st = sampler.status()
    assert st.flags == 0
    assert st.handovers == int(below.sum())
    o = oracle.sample_batch(w.logits, prm, w.rng_seeds, w.hist, w.hist_offsets, V=w.V)
    assert np.array_equal(ids.cpu().numpy().view(np.uint32), o.ids)


def test_status_is_read_once_and_stale_flags_do_not_fail_a_host_call(sampler):
    sampler.status()
    sampler.debug(smp.DEBUG_SET_FLAGS, smp.KSTATUS_SYNC_TIMEOUT)
    w = make_workload(2, B=8)
    # The host entry reports only its own kernels' flags.
    g = sampler.sample_host(w.logits, w.params, w.rng_seeds, w.hist, w.hist_offsets, V=w.V)
    assert g.ids.size == 8
    st = sampler.status()
    assert st.flags == smp.KSTATUS_SYNC_TIMEOUT
    assert sampler.status().flags == 0  # cleared by the read


def test_timed_out_waits_are_reported_and_the_kernels_finish(sampler):
    """One spin per wait. The full-vocabulary kernel's replay wave always
    waits for the other waves' tie split on config 4's rows, so that wait
    runs out. The call must still finish (no hang, no split workgroup) and
    report the timeout, through the host entry's status and through
    llmhip_ctx_status for the device entry."""
    from oracle import oracle

    w = make_workload(4, B=64)
    sampler.status()
    sampler.debug(smp.DEBUG_SPIN_LIMIT, 1)
    try:
        with pytest.raises(smp.SamplerError) as e:
            sampler.sample_host(w.logits, w.params, w.rng_seeds, V=w.V)
        assert e.value.status == -3
        _device_call(sampler, w)
        assert sampler.status().flags & smp.KSTATUS_SYNC_TIMEOUT
    finally:
        sampler.debug(smp.DEBUG_SPIN_LIMIT, 0)
    # Back to the default bound: clean again, and the ids are the oracle's.
    g = sampler.sample_host(w.logits, w.params, w.rng_seeds, V=w.V)
    o = oracle.sample_batch(w.logits, w.params, w.rng_seeds, V=w.V, threads=8)
    assert np.array_equal(g.ids, o.ids)
    assert sampler.status().flags == 0


def test_register_path_with_one_spin_per_wait(sampler):
    """The register kernel's waits (for the threshold, for the history
    counts) are usually over before a wave gets to them. With one spin per
    wait a call either reports a timeout or returns the oracle's ids."""
    from oracle import oracle

    w = make_workload(3, B=256)
    sampler.status()
    sampler.debug(smp.DEBUG_SPIN_LIMIT, 1)
    try:
        try:
            g = sampler.sample_host(w.logits, w.params, w.rng_seeds, w.hist, w.hist_offsets, V=w.V)
        except smp.SamplerError as e:
            assert e.status == -3
        else:
            o = oracle.sample_batch(w.logits, w.params, w.rng_seeds, w.hist, w.hist_offsets, V=w.V, threads=8)
            assert np.array_equal(g.ids, o.ids)
    finally:
        sampler.debug(smp.DEBUG_SPIN_LIMIT, 0)
    sampler.status()


def test_full_vocab_rows_report_their_handovers(sampler):
    """Rows with a NaN go to the sorting path from the full-vocabulary kernel."""
    from oracle import oracle

    rs = np.random.default_rng(5)
    B, V = 8, 4096
    x = rs.standard_normal((B, V)).astype(np.float32)
    x[3, 17] = np.inf
    prm = make_params(1.0, 0, 0.9, 0.0, 1.0)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)
    sampler.status()
    g = sampler.sample_host(x, prm, seeds, V=V)
    st = sampler.status()
    assert st.handovers == 1
    o = oracle.sample_batch(x, prm, seeds, None, None, V=V)
    assert np.array_equal(g.ids, o.ids)
