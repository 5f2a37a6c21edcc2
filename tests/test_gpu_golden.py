"""Token-exact greedy decoding on the GPU against the committed oracle
fixtures (64 steps), through the C ABI's host-driven and device-chained
loops. The fixtures record each step's top-2 logit gap; steps closer than
1e-4 of the top logit are reported instead of judged."""
import pytest

from golden_util import compare_tokens, load, model_of, weights_sha256

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["smoke_q4_seed3_greedy64.json", "smollm3_q4_seed0_greedy64.json"])
def test_greedy_64_matches_fixture(ctx, pkg, name):
    print(f"case golden {name}", flush=True)
    fx = load(name)
    w = model_of(pkg, fx)
    assert weights_sha256(w) == fx["weights_sha256"]
    steps = len(fx["greedy_tokens"])
    be = pkg.HipBackend(ctx, w, kv_capacity=len(fx["prompt"]) + steps + 8)
    got = pkg.generate_greedy_host(be, fx["prompt"], steps)
    assert compare_tokens(fx, got) == steps
    be.kv_reset()
    _, first = be.raw_prefill(fx["prompt"], want_logits=False)
    chained = [first] + be.generate_greedy(first, steps - 1).tolist()
    assert compare_tokens(fx, chained) == steps
