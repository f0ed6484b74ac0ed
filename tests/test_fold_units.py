"""The two facts the full-vocabulary kernel (scriptonait_amd/csrc/vocab_row.h)
and the LDS tail's block folds (scriptonait_amd/csrc/draw_tail.h) rest on,
checked on the CPU.

1. x = expf(w - max) is monotone: glibc's expf is non-decreasing over every
   binary32 input in [-104, 0] (below that it is 0). With w - max and p = x / S
   monotone too, sorting by (w desc, id asc) sorts the terms of every fold of
   crates/llm-core/src/generate.rs:372-419 in descending order, so each fold is
   a fold over a value multiset.

2. While an f32 left fold F stays inside one binade [2^E, 2^(E+1)), a step
   F + t rounds to F + rne(t / u) * u with u = 2^(E-23): an integer count of
   ulps, independent of where t comes in the order, except at an exact
   half-ulp tie, where round-half-even takes the parity of F's last bit
   (ulp count q + ((M ^ q) & 1) for F = M * u). The same rule holds for the
   walk's subtractions (generate.rs:412-419) while F - t stays in the binade.
   Checked against numpy's f32 arithmetic on random and on constructed tie
   cases; a rule that ignores the tie parity must fail.
"""
import subprocess
import textwrap

import numpy as np

MONO = textwrap.dedent(r"""
    #include <math.h>
    #include <stdint.h>
    #include <stdio.h>
    #include <string.h>
    int main(void) {
      unsigned long bad = 0; float prev = 0.0f;
      /* negative floats: bits 0xC2D00000 (-104) up to 0x80000000 (-0) is increasing x */
      for (uint32_t b = 0xC2D00000u;; --b) {
        float x; memcpy(&x, &b, 4);
        const float y = expf(x);
        if (y < prev) ++bad;
        prev = y;
        if (b == 0x80000000u) break;
      }
      printf("%lu\n", bad);
      return 0;
    }
""")


def test_glibc_expf_is_monotone_on_the_softmax_domain(tmp_path):
    src = tmp_path / "mono.c"
    src.write_text(MONO)
    exe = tmp_path / "mono"
    subprocess.run(["gcc", "-O2", str(src), "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120).stdout
    assert int(out) == 0


def _units(F):
    b = np.asarray(F, dtype=np.float32).view(np.uint32).astype(np.int64)
    E = ((b >> 23) & 255) - 127
    M = (b & 0x7FFFFF) | 0x800000
    return E, M


def _rne_units(t, E):
    """t / 2^(E-23) rounded to nearest (q), with exact half-way cases flagged."""
    v = t.astype(np.float64) * np.ldexp(1.0, (23 - E).astype(np.int64))
    q = np.floor(v)
    f = v - q
    return q.astype(np.int64) + (f > 0.5), f == 0.5


def _fold_step(F, t, sub, use_parity=True):
    E, M = _units(F)
    q, tie = _rne_units(t, E)
    d = q + np.where(tie & use_parity, (M ^ q) & 1, 0)
    Mn = M - d if sub else M + d
    return E, Mn


def _check(F, t, sub, use_parity=True):
    E, Mn = _fold_step(F, t, sub, use_parity)
    ref = (F - t if sub else F + t).astype(np.float32)
    inside = (Mn >= (1 << 23) + (1 if sub else 0)) & (Mn < (1 << 24))
    got = np.ldexp(Mn.astype(np.float64), (E - 23).astype(np.int64)).astype(np.float32)
    return inside, got, ref


def test_integer_ulp_steps_match_f32_adds_and_subtractions():
    rs = np.random.default_rng(1)
    n = 400000
    F = (rs.uniform(1, 2, n) * np.ldexp(1.0, rs.integers(-20, 20, n))).astype(np.float32)
    # terms from just below the binade down to far below half an ulp
    t = (F.astype(np.float64) * np.ldexp(1.0, -rs.integers(1, 30, n)) * rs.uniform(0.5, 1.0, n)).astype(np.float32)
    for sub in (False, True):
        inside, got, ref = _check(F, t, sub)
        assert inside.mean() > 0.5
        assert np.array_equal(got[inside], ref[inside]), sub


def test_half_ulp_ties_follow_the_parity_of_the_running_value():
    rs = np.random.default_rng(2)
    n = 200000
    E = rs.integers(-10, 10, n)
    M = rs.integers((1 << 23) + (1 << 13), (1 << 24) - (1 << 13), n)
    F = np.ldexp(M.astype(np.float64), E - 23).astype(np.float32)
    q = rs.integers(0, 1 << 12, n)
    t = np.ldexp((q * 2 + 1).astype(np.float64), E - 23 - 1).astype(np.float32)  # exactly q + 1/2 ulps
    for sub in (False, True):
        inside, got, ref = _check(F, t, sub)
        assert inside.all()
        assert np.array_equal(got, ref), sub
        # Without the parity rule about half of these come out wrong.
        _, bad, _ = _check(F, t, sub, use_parity=False)
        assert (bad != ref).mean() > 0.3


def test_a_fold_of_one_binade_is_order_free_apart_from_ties():
    """Summing the ulp counts of a shuffled run gives the sequential f32 fold."""
    rs = np.random.default_rng(3)
    for _ in range(200):
        F0 = np.float32(rs.uniform(1, 2) * 2.0 ** rs.integers(-5, 5))
        t = (F0 * np.ldexp(1.0, -rs.integers(8, 26, 300)) * rs.uniform(0.5, 1, 300)).astype(np.float32)
        t = np.sort(t)[::-1]
        F = F0
        for x in t:
            F = np.float32(F + x)
        E, M = _units(F0)
        q, tie = _rne_units(t, np.full(t.size, E))
        if tie.any() or _units(F)[0] != E:
            continue
        Mn = M + q[rs.permutation(t.size)].sum()
        assert np.float32(np.ldexp(float(Mn), int(E) - 23)) == F


def test_a_subtraction_that_lands_on_the_binade_floor_can_round_below_it():
    """Why the walk's integer steps need their result a whole ulp above 2^E
    (M - q > 2^23, as `_check` and the LDS tail's walk require): with
    F = 2^E + u and t between u and 1.5 u, rne(t / u) = 1 puts the rule's
    result on 2^E exactly, but F - t lies below 2^E, where the spacing is
    u / 2, and rounds to 2^E - u / 2 once it is closer to that."""
    E = np.arange(-20, 20)
    u = np.ldexp(1.0, E - 23)
    F = np.ldexp(float((1 << 23) + 1), E - 23).astype(np.float32)
    t = (1.4 * u).astype(np.float32)
    _, Mn = _fold_step(F, t, sub=True)
    assert (Mn == (1 << 23)).all()  # the rule lands on 2^E ...
    ref = (F - t).astype(np.float32)
    assert (ref == (np.ldexp(1.0, E) - u / 2).astype(np.float32)).all()  # ... f32 rounds below it
    inside, _, _ = _check(F, t, sub=True)
    assert not inside.any()
