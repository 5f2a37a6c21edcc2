"""The committed greedy fixtures against the generator and the oracle (CPU)."""
import numpy as np

from golden_util import load, model_of, weights_sha256


def test_smoke_fixture_reproduces(pkg, orc):
    fx = load("smoke_q4_seed3_greedy64.json")
    w = model_of(pkg, fx)
    assert weights_sha256(w) == fx["weights_sha256"]
    om = orc.OracleModel(w, kv_capacity=len(fx["prompt"]) + 72, T=4)
    tokens, _ = om.greedy(fx["prompt"], len(fx["greedy_tokens"]))
    assert tokens == fx["greedy_tokens"]


def test_smollm3_fixture_reproduces(pkg, orc):
    """The SmolLM3-3B synthetic model (1.73 GB of Q4 weights): its bytes hash
    to the fixture, and the oracle's first 8 greedy tokens match it."""
    fx = load("smollm3_q4_seed0_greedy64.json")
    w = model_of(pkg, fx)
    assert weights_sha256(w) == fx["weights_sha256"]
    om = orc.OracleModel(w, kv_capacity=len(fx["prompt"]) + 16, T=8)
    tokens, _ = om.greedy(fx["prompt"], 8)
    assert tokens == fx["greedy_tokens"][:8]
    assert min(np.array(fx["top2_gap"]) / np.abs(fx["top_logit"])) > 1e-4   # no near-ties in the fixture
