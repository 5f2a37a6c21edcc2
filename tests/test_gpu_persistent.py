"""The opt-in persistent decode step (one launch per token, QORA_HIP_DECODE=mk
at model set-up) against the oracle and the 64-token greedy fixtures, like
the default graph path."""
import numpy as np
import pytest

import __graft_entry__ as entry
from golden_util import compare_tokens, load, model_of, weights_sha256
from helpers import REL_TOL, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture
def mk(monkeypatch):
    monkeypatch.setenv("QORA_HIP_DECODE", "mk")


def small_model(pkg, layers=4, seed=0):
    cfg = entry.smoke_config(pkg)
    cfg.num_layers = layers
    return pkg.synthetic_model(cfg, seed=seed, fmt=1, rope_positions=128)


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_persistent_prefill_decode_match_oracle(ctx, pkg, orc, mk, kv_dtype):
    print(f"case persistent small model kv_dtype={kv_dtype}", flush=True)
    w = small_model(pkg)
    prompt = pkg.synth_tokens(0, 2000, 13, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128, kv_dtype=kv_dtype)
    assert be.decode_mode() == 2
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    tol = REL_TOL if kv_dtype == 0 else 5e-3   # f16 cache rounding
    logits, tok = be.raw_prefill(prompt)
    ref = om.prefill(prompt)
    assert rel_err(logits, ref) <= tol
    if kv_dtype == 0:
        for layer in (0, 3):
            k, v = be.kv_layer(layer)
            kr, vr = om.kv_layer(layer)
            assert rel_err(k, kr) <= REL_TOL and rel_err(v, vr) <= REL_TOL
    for t in pkg.synth_tokens(0, 2001, 40, w.config.vocab):
        logits, tok = be.forward_decode_raw(int(t))
        ref = om.forward_decode(int(t))
        assert rel_err(logits, ref) <= tol
        if kv_dtype == 0 and orc.top2_gap(ref) > 1e-4 * float(np.max(np.abs(ref))):
            assert tok == orc.argmax(ref)


@pytest.mark.parametrize("name", ["smoke_q4_seed3_greedy64.json", "smollm3_q4_seed0_greedy64.json"])
def test_persistent_greedy_64_matches_fixture(ctx, pkg, mk, name):
    print(f"case persistent golden {name}", flush=True)
    fx = load(name)
    w = model_of(pkg, fx)
    assert weights_sha256(w) == fx["weights_sha256"]
    steps = len(fx["greedy_tokens"])
    be = pkg.HipBackend(ctx, w, kv_capacity=len(fx["prompt"]) + steps + 8)
    assert be.decode_mode() == 2
    got = pkg.generate_greedy_host(be, fx["prompt"], steps)
    assert compare_tokens(fx, got) == steps
    be.kv_reset()
    _, first = be.raw_prefill(fx["prompt"], want_logits=False)
    chained = [first] + be.generate_greedy(first, steps - 1).tolist()
    assert compare_tokens(fx, chained) == steps


def test_default_is_the_graph_path(ctx, pkg, monkeypatch):
    monkeypatch.delenv("QORA_HIP_DECODE", raising=False)
    be = pkg.HipBackend(ctx, small_model(pkg, layers=1), kv_capacity=32)
    assert be.decode_mode() == 1
