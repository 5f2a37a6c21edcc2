"""Loading and checking the committed greedy fixtures (tests/golden/)."""
import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NEAR_TIE = 1e-4    # a step whose top-2 gap is below NEAR_TIE * |top logit| is reported, not judged


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def model_of(pkg, fx):
    c = fx["config"]
    cfg = pkg.ModelConfig(num_layers=c["num_layers"], vocab=c["vocab"], hidden=c["hidden"],
                          intermediate=c["intermediate"], num_heads=c["num_heads"], num_kv_heads=c["num_kv_heads"],
                          head_dim=c["head_dim"], rope_half_dim=c["rope_half_dim"], rope_theta=c["rope_theta"],
                          rope_positions=fx["rope_positions"])
    w = pkg.synthetic_model(cfg, seed=fx["seed"], rope_positions=fx["rope_positions"])
    mult = fx.get("proj_scale", 1.0)
    if mult != 1.0:
        # every projection's Q4 group scales times mult, rounded to binary16
        for ws in w.layers:
            for wt in ws:
                wt.scales = (wt.scales.view(np.float16).astype(np.float32) * np.float32(mult)).astype(
                    np.float16).view(np.uint16)
    return w


def weights_sha256(w):
    h = hashlib.sha256()
    for ws in w.layers:
        for wt in ws:
            h.update(wt.packed.tobytes())
            h.update(wt.scales.tobytes())
    h.update(w.embed.packed.tobytes())
    h.update(w.embed.scales.tobytes())
    for g in list(w.input_norm) + list(w.post_attn_norm) + [w.final_norm]:
        h.update(g.tobytes())
    h.update(w.rope_cos.tobytes())
    h.update(w.rope_sin.tobytes())
    return h.hexdigest()


def compare_tokens(fx, got):
    """Token-exact up to the first step the fixture marks as a near-tie;
    returns the number of steps compared."""
    want = fx["greedy_tokens"]
    for i, (a, b) in enumerate(zip(got, want)):
        if fx["top2_gap"][i] < NEAR_TIE * abs(fx["top_logit"][i]):
            print(f"step {i}: near-tie in the fixture (gap {fx['top2_gap'][i]:.3g}), comparison stops here")
            return i
        assert a == b, f"step {i}: got token {a}, fixture {b} (gap {fx['top2_gap'][i]:.3g})"
    assert len(got) == len(want)
    return len(want)
