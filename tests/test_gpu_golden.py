"""Token-exact greedy decoding on the GPU against the committed oracle
fixtures, through the C ABI's host-driven and device-chained loops:
- the 8-layer smoke model (64 steps, 48 distinct tokens);
- SmolLM3-3B after a 64-token prompt, 128 steps (positions 64..191, the
  fused short-context attention);
- SmolLM3-3B after a 1920-token prompt (batched prefill in four chunks),
  128 steps at positions 1920..2047 (the split attention past 256
  positions, the 2048-context workload).
The fixtures record each step's top-2 logit gap; steps closer than 1e-4 of
the top logit are reported instead of judged."""
import pytest

from golden_util import compare_tokens, load, model_of, weights_sha256

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["smoke_q4_seed0_x8_greedy64.json", "smollm3_q4_seed0_greedy128.json",
                                  "smollm3_q4_seed0_ctx2048_greedy128.json"])
def test_greedy_matches_fixture(ctx, pkg, name):
    print(f"case golden {name}", flush=True)
    fx = load(name)
    w = model_of(pkg, fx)
    assert weights_sha256(w) == fx["weights_sha256"]
    steps = len(fx["greedy_tokens"])
    be = pkg.HipBackend(ctx, w, kv_capacity=fx["rope_positions"])
    got = pkg.generate_greedy_host(be, fx["prompt"], steps)
    assert compare_tokens(fx, got) == steps
    be.kv_reset()
    _, first = be.raw_prefill(fx["prompt"], want_logits=False)
    chained = [first] + be.generate_greedy(first, steps - 1).tolist()
    assert compare_tokens(fx, chained) == steps
