"""The oracle's sampling restatement (generate.rs:38-91, 345-395) pinned on
the CPU: the xorshift64 Rng against an integer restatement, the first-max and
degenerate cases, the penalties' per-occurrence and window semantics, and the
sampled frequencies against the float64 top-k / top-p distribution."""
import numpy as np
import pytest

M64 = (1 << 64) - 1


def xorshift_int(state, n):
    out = []
    for _ in range(n):
        state ^= (state << 13) & M64
        state ^= state >> 7
        state ^= (state << 17) & M64
        out.append((state >> 40) / 16777216.0)
    return out, state


@pytest.mark.parametrize("seed", [1, 12345, (1 << 63) + 7, 0x9E3779B97F4A7C15])
def test_rng_matches_integer_xorshift(orc, seed):
    want, end = xorshift_int(seed, 50)
    st = seed
    for w in want:
        v, st = orc.rng_next_f32(st)
        assert v == np.float32(w) and 0.0 <= v < 1.0
    assert st == end


def test_greedy_is_first_max_and_ignores_penalties(orc):
    lg = np.array([0.5, 3.0, -1.0, 3.0, 2.0], np.float32)
    tok, st = orc.sample(lg, [1, 1, 1], 0.0, 0.95, 20, 1.1, 1.5, 77)
    assert tok == 1 and st == 77            # no draw, no penalty in greedy mode


def test_degenerate_settings_take_the_top_candidate(orc):
    r = np.random.default_rng(0)
    lg = r.standard_normal(1000).astype(np.float32)
    best = int(np.argmax(lg))
    st = 5
    for _ in range(20):
        t1, st1 = orc.sample(lg, [], 0.8, 0.95, 1, 1.0, 0.0, st)     # top_k = 1
        t2, st2 = orc.sample(lg, [], 0.8, 1e-9, 20, 1.0, 0.0, st)    # nucleus of one
        assert t1 == t2 == best
        assert st1 == st2 == xorshift_int(st, 1)[1]                  # exactly one draw each
        st = st1


def test_penalties_per_occurrence_and_window(orc):
    vocab = 10
    lg = np.array([2.0, -2.0, 1.0, 0.5, 4.0, 0.0, -1.0, 3.0, 1.5, 0.25], np.float32)
    # token 0 three times in the last 64, token 1 twice, token 2 only before the window
    hist = [2] * 10 + [9] * 60 + [0, 1, 0, 1, 0]
    got = lg.copy()
    orc.lib().oq_repetition_penalty(got.ctypes.data, vocab, np.asarray(hist, np.uint32).ctypes.data, len(hist),
                                    np.float32(1.1))
    p = np.float32(1.1)
    assert got[0] == np.float32(np.float32(np.float32(lg[0] / p) / p) / p)
    assert got[1] == np.float32(np.float32(lg[1] * p) * p)
    assert got[2] == lg[2]                  # outside the last 64
    x = lg[9]
    for _ in range(59):                     # indices 11..69 of the history are in the window
        x = np.float32(x / p)
    assert got[9] == x
    pres = lg.copy()
    h = np.asarray(hist, np.uint32)
    orc.lib().oq_presence_penalty(pres.ctypes.data, vocab, h.ctypes.data, len(hist), np.float32(1.5))
    for t in range(vocab):
        assert pres[t] == (np.float32(lg[t] - np.float32(1.5)) if t in hist else lg[t])


@pytest.mark.parametrize("top_k,top_p", [(20, 0.9), (0, 0.93), (1000, 0.93)])
def test_sampled_frequencies_match_float64_distribution(orc, top_k, top_p):
    """20000 draws against the distribution the definition fixes: softmax of
    (l - max) / T over the top_k logits (top_k 0 or above the vocabulary: all
    of them, generate.rs:363), cut at the first cumulative mass >= top_p,
    renormalised."""
    r = np.random.default_rng(3)
    lg = (r.standard_normal(300) * 1.5).astype(np.float32)
    T = 0.8
    kk = top_k if 0 < top_k < lg.size else lg.size
    order = np.lexsort((np.arange(lg.size), -lg.astype(np.float64)))[:kk]
    z = np.exp((lg[order].astype(np.float64) - lg.max()) / T)
    pz = z / z.sum()
    cut = int(np.searchsorted(np.cumsum(pz), top_p) + 1)
    assert abs(np.cumsum(pz)[cut - 1] - top_p) > 1e-3          # away from the cut-off boundary
    want = pz[:cut] / pz[:cut].sum()
    counts = np.zeros(lg.size)
    st = 99
    n = 20000
    for _ in range(n):
        tok, st = orc.sample(lg, [], T, top_p, top_k, 1.0, 0.0, st)
        counts[tok] += 1
    assert counts[np.setdiff1d(np.arange(lg.size), order[:cut])].sum() == 0
    freq = counts[order[:cut]] / n
    sigma = np.sqrt(want * (1 - want) / n)
    assert np.all(np.abs(freq - want) <= 5 * sigma + 1e-4)
