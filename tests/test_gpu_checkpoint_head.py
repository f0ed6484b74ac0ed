"""GPU: a checkpoint's tied embedding table through the output head and the
sampler (llmhip_scck_* then llmhip_sample_tied_head_device), against the
oracle's linear_fwd and sample_with on the table the reader returns.

The file is a bf16 checkpoint (what the site ships, checkpoint.rs:26-36)
written by tests/scck_writer.py; the reader widens it as from_bf16 does, and
the table must be bit-identical to the widened stored bits.
"""
import numpy as np
import pytest

from oracle import oracle
from scriptonait_amd.checkpoint import Checkpoint
from scriptonait_amd.workloads import make_params
from tests import scck_writer as W

pytestmark = pytest.mark.gpu


def test_checkpoint_embedding_feeds_the_tied_head(sampler):
    import torch

    V, H, L = 264 + 4000, 64, 1
    w = W.sample_weights(vocab_size=V, hidden_dim=H, num_layers=L, num_heads=4, num_kv_heads=2, seed=9)
    w[: V * H] *= 10.0  # a peakier head than the init scale, so the filters cut
    data = W.write(w, num_layers=L, hidden_dim=H, num_heads=4, num_kv_heads=2, context_len=64, local_window=32,
                   vocab_size=V, bf16=True)
    ck = Checkpoint.from_bytes(data)
    embed = ck.embed()
    assert embed.shape == (V, H)
    assert np.array_equal(embed.view(np.uint32), W.to_bf16(w[: V * H]).astype(np.uint32).reshape(V, H) << 16)

    rs = np.random.default_rng(21)
    B = 48
    hidden = rs.standard_normal((B, H)).astype(np.float32) * ck.final_norm_gain()[None, :] * 50.0
    prm = make_params(0.8, 40, 0.95, 0.05, 1.1)
    Hh = 200
    hist = rs.integers(0, V, size=B * Hh).astype(np.uint32)
    offs = (np.arange(B + 1) * Hh).astype(np.uint32)
    seeds = rs.integers(0, 2**63, size=B, dtype=np.uint64)

    dev = torch.device("cuda:0")
    rng = torch.from_numpy(seeds.view(np.int64).copy()).to(dev)
    ids = torch.zeros(B, dtype=torch.int32, device=dev)
    kept = torch.zeros(B, dtype=torch.int32, device=dev)
    lg = torch.zeros((B, V), dtype=torch.float32, device=dev)
    sampler.sample_tied_head_device(torch.from_numpy(hidden).to(dev), torch.from_numpy(embed).to(dev), prm, rng, ids,
                                    hist=torch.from_numpy(hist.view(np.int32)).to(dev),
                                    hist_offsets=torch.from_numpy(offs.view(np.int32)).to(dev), out_kept=kept,
                                    out_logits=lg)
    torch.cuda.synchronize()
    want = oracle.linear_fwd(hidden, embed, threads=8)
    assert np.all(lg.cpu().numpy() == want)
    o = oracle.sample_batch(want, prm, seeds, hist, offs, V=V, threads=8)
    assert np.array_equal(ids.cpu().numpy().view(np.uint32), o.ids)
    assert np.array_equal(rng.cpu().numpy().view(np.uint64), o.rng_state)
    assert np.array_equal(kept.cpu().numpy().view(np.uint32), o.kept)
    assert np.all(o.kept > 1)  # the filters kept more than one candidate: a real draw
