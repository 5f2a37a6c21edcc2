"""The committed greedy fixtures against the generator and the oracle (CPU)."""
import numpy as np
import pytest

from golden_util import NEAR_TIE, load, model_of, weights_sha256

SMOKE = "smoke_q4_seed0_x8_greedy64.json"
SMOLLM3 = ("smollm3_q4_seed0_greedy128.json", "smollm3_q4_seed0_ctx2048_greedy128.json")


def test_smoke_fixture_reproduces(pkg, orc):
    fx = load(SMOKE)
    w = model_of(pkg, fx)
    assert weights_sha256(w) == fx["weights_sha256"]
    om = orc.OracleModel(w, kv_capacity=len(fx["prompt"]) + 72, T=4)
    tokens, _ = om.greedy(fx["prompt"], len(fx["greedy_tokens"]))
    assert tokens == fx["greedy_tokens"]


def test_smoke_fixture_discriminates():
    """The smoke fixture's greedy path visits many distinct tokens, so a
    token comparison tests every step, not only the first."""
    fx = load(SMOKE)
    assert len(set(fx["greedy_tokens"])) >= 32
    assert min(np.array(fx["top2_gap"]) / np.abs(fx["top_logit"])) > NEAR_TIE


@pytest.mark.parametrize("name", SMOLLM3)
def test_smollm3_fixture_reproduces(pkg, orc, name):
    """The SmolLM3-3B synthetic model (1.73 GB of Q4 weights): its bytes hash
    to the fixture, its prompt is the seeded one, and the oracle's first 4
    greedy tokens after the prompt match it (the whole fixture took minutes
    of oracle time to write; the GPU tests compare every step)."""
    fx = load(name)
    w = model_of(pkg, fx)
    assert weights_sha256(w) == fx["weights_sha256"]
    assert fx["prompt"] == pkg.synth_tokens(fx["seed"], fx["prompt_tid"], len(fx["prompt"]), w.config.vocab).tolist()
    assert len(fx["greedy_tokens"]) == 128
    if len(fx["prompt"]) <= 64:
        om = orc.OracleModel(w, kv_capacity=len(fx["prompt"]) + 16, T=8)
        tokens, _ = om.greedy(fx["prompt"], 4)
        assert tokens == fx["greedy_tokens"][:4]
    assert min(np.array(fx["top2_gap"]) / np.abs(fx["top_logit"])) > NEAR_TIE   # no near-ties in the fixture
    assert len(set(fx["greedy_tokens"])) >= 8
