"""CPU: the checkpoint reader (llmhip_scck_parse / llmhip_scck_read_params
through scriptonait_amd.checkpoint) against crates/llm-core/src/checkpoint.rs.

The reference's own checkpoint tests (checkpoint.rs:292-420) are ported:
round trip, version 2 and 3 files, bf16 size and closeness, truncated,
foreign and inconsistent files. Files are written by tests/scck_writer.py
(a restatement of write_checkpoint). The header layout is pinned by the
reference tests' own offsets (step at 8 + 7*4 + 4 + 4), and
ModelConfig::validate's rules (config.rs:169-217) each get a rejected file.
"""
import struct

import numpy as np
import pytest

from scriptonait_amd.checkpoint import Checkpoint
from tests import scck_writer as W

V, H = 320, 16  # the reference test's tokenizer trains to 320 ids; hidden 16


def _sample(**kw):
    w = W.sample_weights(vocab_size=kw.get("vocab_size", V), hidden_dim=H)
    return w, W.write(w, vocab_size=kw.pop("vocab_size", V), **kw)


def test_round_trips():
    w, data = _sample()
    c = Checkpoint.from_bytes(data)
    assert (c.config.num_layers, c.config.hidden_dim, c.config.num_heads, c.config.num_kv_heads) == (2, 16, 4, 2)
    assert (c.config.context_len, c.config.local_window, c.config.vocab_size) == (32, 16, V)
    assert c.config.rope_theta == 50000.0 and c.config.use_ple is False
    assert (c.step, c.tokens_seen, c.planned_steps, c.plateau_scale) == (4242, 9_000_000, 23_000, 0.5)
    assert c.num_merges == V - 264 and c.weight_dtype == "f32"
    assert c.param_count == w.size
    assert np.array_equal(c.params(0, w.size), w)
    assert np.array_equal(c.embed(), w[: V * H].reshape(V, H))
    assert np.array_equal(c.final_norm_gain(), w[-H:])
    assert np.array_equal(c.params(123, 77), w[123:200])


def test_a_version_2_checkpoint_still_loads():
    _, data = _sample()
    b = bytearray(data)
    b[4:8] = struct.pack("<I", 2)
    step_at = 8 + 7 * 4 + 4 + 4
    del b[step_at + 8: step_at + 8 + 8 + 4 + 4]
    c = Checkpoint.from_bytes(bytes(b))
    assert (c.step, c.tokens_seen, c.planned_steps, c.plateau_scale) == (4242, 0, 0, 1.0)


def test_a_version_3_checkpoint_still_loads():
    _, data = _sample()
    b = bytearray(data)
    b[4:8] = struct.pack("<I", 3)
    tokens_seen_at = 8 + 7 * 4 + 4 + 4 + 8
    del b[tokens_seen_at + 8: tokens_seen_at + 8 + 4 + 4]
    c = Checkpoint.from_bytes(bytes(b))
    assert (c.step, c.tokens_seen, c.planned_steps, c.plateau_scale) == (4242, 9_000_000, 0, 1.0)


def test_the_writer_versions_match_the_reference_cuts():
    """tests/scck_writer.py's version-2/3 files are the reference tests' cut
    version-4 files, byte for byte."""
    w, v4 = _sample()
    for version, cut_at, cut in ((2, 8 + 7 * 4 + 4 + 4 + 8, 16), (3, 8 + 7 * 4 + 4 + 4 + 16, 8)):
        b = bytearray(v4)
        b[4:8] = struct.pack("<I", version)
        del b[cut_at: cut_at + cut]
        assert bytes(b) == W.write(w, vocab_size=V, version=version)


def test_bf16_checkpoints_are_half_the_size_and_close_enough():
    w, f32 = _sample()
    _, bf = _sample(bf16=True)
    assert len(bf) < len(f32) * 3 // 5
    c = Checkpoint.from_bytes(bf)
    assert c.weight_dtype == "bf16" and c.step == 4242
    got = c.params(0, w.size)
    assert np.max(np.abs(got - w)) < 0.01
    # from_bf16: the stored 16 bits are the top of the f32, the rest zero
    assert np.array_equal(got.view(np.uint32), W.to_bf16(w).astype(np.uint32) << 16)


def test_rejects_a_truncated_file():
    _, data = _sample()
    for cut in (0, 4, 20, len(data) // 2, len(data) - 1):
        with pytest.raises(ValueError):
            Checkpoint.from_bytes(data[:cut])


def test_rejects_a_foreign_file():
    with pytest.raises(ValueError, match="not a scriptonait checkpoint"):
        Checkpoint.from_bytes(b"not a checkpoint at all")


def test_rejects_a_tokenizer_that_does_not_match_the_config():
    w = W.sample_weights(vocab_size=V + 1, hidden_dim=H)
    data = W.write(w, vocab_size=V + 1, tokenizer=W.tokenizer_bytes(V - 264))
    with pytest.raises(ValueError, match="inconsistent"):
        Checkpoint.from_bytes(data)


@pytest.mark.parametrize(
    "change,match",
    [
        (dict(num_layers=0), "num_layers"),
        (dict(hidden_dim=6, num_heads=2), "hidden_dim"),
        (dict(num_heads=3), "divide"),                       # 16 % 3 != 0
        (dict(num_heads=16, num_kv_heads=16), "even"),       # head_dim 1
        (dict(num_kv_heads=3), "divide"),                    # 4 % 3 != 0
        (dict(context_len=1), "context_len"),
        (dict(local_window=0), "local_window"),
        (dict(rope_theta=1.0), "rope_theta"),
        (dict(version=5), "version"),
        (dict(version=1), "version"),
    ],
)
def test_rejects_an_invalid_header(change, match):
    _, data = _sample(**change)
    with pytest.raises(ValueError, match=match):
        Checkpoint.from_bytes(data)


def test_rejects_a_config_too_big_to_train():
    """config.rs:453-460's shape (16 layers, 1024 wide, 16 heads, 4096-token
    attention) needs ~20 GB to train: rejected before the weights are read."""
    hdr = bytearray(b"SCCK") + struct.pack("<I", 4) + struct.pack("<7I", 16, 1024, 16, 16, 4096, 4096, 264)
    hdr += struct.pack("<fI", 10000.0, 0) + bytes(64)
    with pytest.raises(ValueError, match="train"):
        Checkpoint.from_bytes(bytes(hdr))


def test_rejects_bad_tokenizers_and_weights():
    w = W.sample_weights(vocab_size=V, hidden_dim=H)
    tok = bytearray(W.tokenizer_bytes(V - 264))
    bad_merge = bytearray(tok)
    bad_merge[12:16] = struct.pack("<I", 264)  # merge 0 may only use ids < 264
    with pytest.raises(ValueError, match="merge 0"):
        Checkpoint.from_bytes(W.write(w, vocab_size=V, tokenizer=bytes(bad_merge)))
    bad_ver = bytearray(tok)
    bad_ver[4:8] = struct.pack("<I", 2)
    with pytest.raises(ValueError, match="tokenizer format version"):
        Checkpoint.from_bytes(W.write(w, vocab_size=V, tokenizer=bytes(bad_ver)))
    with pytest.raises(ValueError, match="bytes for this config"):
        Checkpoint.from_bytes(W.write(w[:-1], vocab_size=V))
    data = bytearray(W.write(w, vocab_size=V))
    dtype_at = 8 + 7 * 4 + 4 + 4 + 8 + 8 + 4 + 4
    data[dtype_at: dtype_at + 4] = struct.pack("<I", 2)
    with pytest.raises(ValueError, match="dtype"):
        Checkpoint.from_bytes(bytes(data))
    # bf16 weights of an odd byte count
    bf = bytearray(W.write(w, vocab_size=V, bf16=True))
    wlen_at = len(bf) - w.size * 2 - 4
    assert struct.unpack("<I", bf[wlen_at: wlen_at + 4])[0] == w.size * 2
    odd = bf[:wlen_at] + struct.pack("<I", w.size * 2 - 1) + bf[wlen_at + 4: -1]
    with pytest.raises(ValueError, match="odd"):
        Checkpoint.from_bytes(bytes(odd))


def test_read_params_rejects_ranges_past_the_end():
    w, data = _sample()
    c = Checkpoint.from_bytes(data)
    with pytest.raises(ValueError):
        c.params(w.size - 3, 4)
    assert c.params(w.size, 0).size == 0


def test_accepts_a_nan_rope_theta_as_the_reference_does():
    """config.rs:209 rejects `rope_theta <= 1.0`; NaN compares false there, so
    Checkpoint::from_bytes accepts the file, and so does the reader."""
    _, data = _sample(rope_theta=float("nan"))
    got = Checkpoint.from_bytes(data)
    assert np.isnan(got.config.rope_theta)
    assert got.config.vocab_size == V
