"""On-device sampling (qora_hip_sample, qora_hip_decode_sample) against the
oracle's restatement of generate.rs:38-91, 345-395 on the same logits: the
same token and the same Rng state, draw for draw."""
import ctypes

import numpy as np
import pytest

import __graft_entry__ as entry
from helpers import device

pytestmark = pytest.mark.gpu

SETTINGS = [
    dict(temperature=0.7, top_p=0.95, top_k=20, repetition_penalty=1.1, presence_penalty=1.5),   # main.rs defaults
    dict(temperature=1.3, top_p=1.0, top_k=64, repetition_penalty=1.0, presence_penalty=0.0),
    dict(temperature=0.35, top_p=0.5, top_k=5, repetition_penalty=1.3, presence_penalty=0.0),
    dict(temperature=0.0, top_p=0.95, top_k=20, repetition_penalty=1.1, presence_penalty=1.5),   # greedy
    dict(temperature=0.9, top_p=0.95, top_k=1, repetition_penalty=1.1, presence_penalty=0.5),
]


@pytest.mark.parametrize("vocab", [128256, 1000, 4097])
@pytest.mark.parametrize("si", range(len(SETTINGS)))
def test_sample_matches_oracle(ctx, pkg, orc, vocab, si):
    sp = SETTINGS[si]
    print(f"case sample vocab={vocab} settings={si}", flush=True)
    r = np.random.default_rng(vocab + si)
    params = pkg.SampleParams(**sp)
    st_gpu = st_orc = 0x2545F4914F6CDD1D + si
    with device(ctx) as d:
        for trial in range(40):
            lg = (r.standard_normal(vocab) * 2.5).astype(np.float32)
            hist = r.integers(0, vocab, size=int(r.integers(0, 150))).tolist()
            hist += hist[-5:] * 2                 # repeats inside the last-64 window
            dl = d.put(lg)
            tok, st_gpu = ctx.sample(dl, vocab, hist, params, st_gpu)
            want, st_orc = orc.sample(lg, hist, sp["temperature"], sp["top_p"], sp["top_k"],
                                      sp["repetition_penalty"], sp["presence_penalty"], st_orc)
            assert tok == want, trial
            assert st_gpu == st_orc


def test_sample_ties_and_zero_signs(ctx, pkg, orc):
    vocab = 3000
    lg = np.full(vocab, -5.0, np.float32)
    lg[[2999, 17, 2048, 700]] = 4.0                 # four-way tie for the maximum
    lg[5] = -0.0
    lg[6] = 0.0
    greedy = pkg.SampleParams(temperature=0.0, top_p=0.95, top_k=20, repetition_penalty=1.1, presence_penalty=1.5)
    top1 = pkg.SampleParams(temperature=0.8, top_p=0.95, top_k=1, repetition_penalty=1.0, presence_penalty=0.0)
    with device(ctx) as d:
        dl = d.put(lg)
        assert ctx.sample(dl, vocab, [], greedy, 9)[0] == 17
        assert ctx.sample(dl, vocab, [], top1, 9)[0] == 17
        st = 11
        for _ in range(30):
            sp = dict(temperature=2.0, top_p=1.0, top_k=6, repetition_penalty=1.0, presence_penalty=0.0)
            tok, st2 = ctx.sample(dl, vocab, [], pkg.SampleParams(**sp), st)
            want, st3 = orc.sample(lg, [], 2.0, 1.0, 6, 1.0, 0.0, st)
            assert tok == want and st2 == st3
            st = st2


def test_sample_errors(ctx, pkg):
    with device(ctx) as d:
        dl = d.put(np.zeros(16, np.float32))
        ok = pkg.SampleParams(temperature=0.7, top_p=0.9, top_k=20, repetition_penalty=1.0, presence_penalty=0.0)
        with pytest.raises(pkg.QoraHipError):
            ctx.sample(dl, 0, [], ok, 1)                # empty vocabulary
        with pytest.raises(pkg.QoraHipError):
            ctx.sample(dl, (1 << 22) + 1, [], ok, 1)    # beyond the supported vocabulary


# the full-sort path: top_k 0 (the whole vocabulary), top_k above 64, a
# vocabulary above 131072 (generate.rs:357-363)
SORT_CASES = [(1000, 0), (4097, 100), (128256, 0), (128256, 1000), (200000, 20), (5000, 6000)]


@pytest.mark.parametrize("vocab,top_k", SORT_CASES)
def test_sample_full_sort_matches_oracle(ctx, pkg, orc, vocab, top_k):
    print(f"case sample full sort vocab={vocab} top_k={top_k}", flush=True)
    r = np.random.default_rng(vocab + top_k)
    settings = [dict(temperature=0.9, top_p=0.95, repetition_penalty=1.1, presence_penalty=1.5),
                dict(temperature=1.4, top_p=1.0, repetition_penalty=1.0, presence_penalty=0.0),
                dict(temperature=0.0, top_p=0.95, repetition_penalty=1.1, presence_penalty=0.0)]
    with device(ctx) as d:
        for si, sp in enumerate(settings):
            params = pkg.SampleParams(top_k=top_k, **sp)
            st_gpu = st_orc = 0x9E3779B97F4A7C15 + si
            for trial in range(8):
                lg = (r.standard_normal(vocab) * 2.5).astype(np.float32)
                if trial == 6:
                    # every logit equal: the sums are whole numbers, crossing a
                    # binade at every power of two
                    lg[:] = 0.5
                if trial == 7:
                    # two levels: long runs of equal terms
                    lg = np.where(r.random(vocab) < 0.3, 1.0, -2.0).astype(np.float32)
                if trial == 1:
                    lg[r.integers(0, vocab, size=50)] = lg.max()     # ties at the top
                if trial in (2, 3):
                    # peaked distributions: most probabilities fall far
                    # below half an ulp of the running sums
                    lg *= 4.0 if trial == 2 else 12.0
                hist = r.integers(0, vocab, size=int(r.integers(0, 100))).tolist()
                dl = d.put(lg)
                tok, st_gpu = ctx.sample(dl, vocab, hist, params, st_gpu)
                want, st_orc = orc.sample(lg, hist, sp["temperature"], sp["top_p"], top_k,
                                          sp["repetition_penalty"], sp["presence_penalty"], st_orc)
                assert tok == want, (si, trial)
                assert st_gpu == st_orc


def test_decode_sample_matches_decode_plus_oracle_sampling(ctx, pkg, orc):
    """A sampled generation on the device equals, token for token, the decode
    step's logits sampled by the oracle with the same Rng stream."""
    cfg = entry.smoke_config(pkg)
    w = pkg.synthetic_model(cfg, seed=5, rope_positions=64)
    prompt = pkg.synth_tokens(5, 2000, 9, cfg.vocab)
    sp = dict(temperature=0.9, top_p=0.95, top_k=20, repetition_penalty=1.1, presence_penalty=1.5)
    params = pkg.SampleParams(**sp)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    _, tok = be.raw_prefill(prompt, want_logits=False)
    hist, st, toks = [tok], 4242, []
    for _ in range(24):
        logits, nxt, st_new = be.decode_sample(hist[-1], hist, params, st, want_logits=True)
        want, st_want = orc.sample(logits, hist, sp["temperature"], sp["top_p"], sp["top_k"],
                                   sp["repetition_penalty"], sp["presence_penalty"], st)
        assert nxt == want and st_new == st_want
        hist.append(nxt)
        st = st_new
    assert be.kv_len() == len(prompt) + 24


def test_decode_sample_refused_call_launches_nothing(ctx, pkg, orc):
    """decode_sample refused for its arguments (no sampling parameters) checks
    them before the step is launched: the cache length is unchanged, and the
    greedy steps that follow match the oracle."""
    print("case refused decode_sample", flush=True)
    cfg = entry.smoke_config(pkg)
    w = pkg.synthetic_model(cfg, seed=6, rope_positions=64)
    prompt = pkg.synth_tokens(6, 2000, 7, cfg.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    om = orc.OracleModel(w, kv_capacity=64, T=4)
    ref_toks, _ = om.greedy(prompt, 6)
    _, tok = be.raw_prefill(prompt, want_logits=False)
    _, tok = be.forward_decode_raw(tok, want_logits=False)     # leaves a logits-free step behind
    got = [ref_toks[0], tok]
    n0 = be.kv_len()
    st = ctypes.c_uint64(7)
    out = ctypes.c_uint32()
    rc = ctx.lib.qora_hip_decode_sample(ctx.h, int(tok), None, 0, None, ctypes.byref(st), None, ctypes.byref(out))
    assert rc == -1
    assert be.kv_len() == n0 and st.value == 7
    for _ in range(4):
        _, tok = be.forward_decode_raw(tok, want_logits=False)
        got.append(tok)
    assert got == ref_toks


@pytest.mark.parametrize("sp", [dict(temperature=0.9, top_p=0.95, top_k=20, repetition_penalty=1.1, presence_penalty=1.5),
                                dict(temperature=1.6, top_p=1.0, top_k=64, repetition_penalty=1.0, presence_penalty=0.0)])
def test_decode_sample_without_logits_matches_with_logits(ctx, pkg, orc, sp):
    """The no-wait path (no logits asked for) gives the same tokens and Rng
    states as the path that returns the logits, which the oracle's sampler
    checks draw for draw; some sampled tokens differ from the greedy token, so
    the next step's token upload is exercised."""
    print(f"case decode_sample no logits t={sp['temperature']}", flush=True)
    cfg = entry.smoke_config(pkg)
    w = pkg.synthetic_model(cfg, seed=7, rope_positions=64)
    prompt = pkg.synth_tokens(7, 2000, 9, cfg.vocab)
    params = pkg.SampleParams(**sp)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    runs = []
    not_greedy = 0
    for want in (True, False):
        _, tok = be.raw_prefill(prompt, want_logits=False)
        hist, st, seen = [tok], 99, []
        for _ in range(20):
            logits, nxt, st_new = be.decode_sample(hist[-1], hist, params, st, want_logits=want)
            if want:
                exp_tok, exp_st = orc.sample(logits, hist, sp["temperature"], sp["top_p"], sp["top_k"],
                                             sp["repetition_penalty"], sp["presence_penalty"], st)
                assert nxt == exp_tok and st_new == exp_st
                not_greedy += int(nxt != orc.argmax(logits))
            seen.append((nxt, st_new))
            hist.append(nxt)
            st = st_new
        runs.append(seen)
    assert runs[0] == runs[1]
    assert not_greedy > 0
