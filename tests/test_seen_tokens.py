"""The allowed mask built from a corpus's tokens (Corpus::seen_tokens,
crates/llm-core/src/corpus.rs:236-247) and its bit layout, on the CPU: the
oracle's restatement against a loop that follows the reference line by line,
and known answers for the packed words."""
import numpy as np

from oracle import oracle


def _seen_loop(token_lists, vocab_size):
    # corpus.rs:236-247: vec![false; vocab_size]; for each id of each source,
    # seen.get_mut(id) -> Some(flag) only for id < vocab_size.
    seen = [False] * vocab_size
    for tokens in token_lists:
        for t in tokens:
            if t < vocab_size:
                seen[t] = True
    return np.array(seen, dtype=bool)


def test_seen_tokens_matches_the_reference_loop():
    rs = np.random.default_rng(0)
    for V in (1, 7, 31, 32, 33, 259, 1000):
        lists = [rs.integers(0, V + 40, size=int(rs.integers(0, 60))).tolist() for _ in range(4)]
        flat = np.array([t for l in lists for t in l], dtype=np.uint32)
        assert np.array_equal(oracle.seen_tokens(flat, V), _seen_loop(lists, V)), V


def test_seen_tokens_known_answers():
    assert not oracle.seen_tokens(np.zeros(0, dtype=np.uint32), 259).any()  # empty corpus
    assert oracle.seen_tokens(np.arange(259, dtype=np.uint32), 259).all()
    s = oracle.seen_tokens(np.array([72, 105, 258, 259, 4000000000], dtype=np.uint32), 259)
    assert np.nonzero(s)[0].tolist() == [72, 105, 258]  # ids >= V are skipped


def test_bit_layout_known_words():
    m = np.zeros(70, dtype=bool)
    m[[0, 31, 32, 69]] = True
    w = oracle.pack_bits(m)
    assert w.dtype == np.uint32 and w.tolist() == [0x80000001, 0x00000001, 0x00000020]
    assert np.array_equal(oracle.unpack_bits(w, 70), m)
    rs = np.random.default_rng(1)
    for n in (1, 32, 33, 1000):
        m = rs.random(n) < 0.4
        assert np.array_equal(oracle.unpack_bits(oracle.pack_bits(m), n), m)
