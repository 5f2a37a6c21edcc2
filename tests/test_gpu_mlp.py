"""The fused MLP launch on the GPU (opt-in, QORA_HIP_MLP=1): each layer's
gate|up and down GEMVs in one kernel (gemv_q4m_mlp_kernel), the down
workgroups waiting on arrival counts of the gate|up workgroups. The reference runs the fused gate+up GEMV
and then the down GEMV (gemv.rs:1002-1006 inside forward_decode_raw); both
launches accumulate exact integer sums, so the fused and the two-launch steps
must agree bit for bit, and both match the oracle."""
import numpy as np
import pytest

from helpers import REL_TOL, rel_err

pytestmark = pytest.mark.gpu


def _model(pkg, layers=2, seed=11):
    # SmolLM3 widths (2048 -> 2 x 11008 -> 2048): the plans the fused kernel takes
    cfg = pkg.ModelConfig(num_layers=layers, vocab=1000, hidden=2048, intermediate=11008, num_heads=16,
                          num_kv_heads=4, head_dim=128, rope_half_dim=64, rope_theta=5e6, rope_positions=128)
    return pkg.synthetic_model(cfg, seed=seed, fmt=1, rope_positions=128)


def _run(pkg, ctx, w, prompt, tokens):
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    fused = be.mlp_fused()
    be.raw_prefill(prompt, want_logits=False)
    out = [be.forward_decode_raw(int(t)) for t in tokens]
    k, v = be.kv_layer(1)
    return fused, out, k, v


def test_fused_and_two_launch_mlp_bit_identical(ctx, pkg, orc, monkeypatch):
    print("case fused mlp vs two launches", flush=True)
    w = _model(pkg)
    prompt = pkg.synth_tokens(11, 2600, 20, w.config.vocab)
    tokens = pkg.synth_tokens(11, 2601, 6, w.config.vocab)
    fused2, out_s, ks, vs = _run(pkg, ctx, w, prompt, tokens)
    assert not fused2                                     # two launches by default
    monkeypatch.setenv("QORA_HIP_MLP", "1")
    fused, out_f, kf, vf = _run(pkg, ctx, w, prompt, tokens)
    assert fused
    for (lf, tf), (ls, ts) in zip(out_f, out_s):
        assert np.array_equal(lf, ls) and tf == ts
    assert np.array_equal(kf, ks) and np.array_equal(vf, vs)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    om.prefill(prompt)
    for t, (lf, _) in zip(tokens, out_f):
        assert rel_err(lf, om.forward_decode(int(t))) <= REL_TOL


def test_fused_mlp_device_chained_greedy(ctx, pkg, orc, monkeypatch):
    """generate_greedy replays the fused step back to back: tokens equal the
    oracle's greedy ones."""
    print("case fused mlp greedy", flush=True)
    monkeypatch.setenv("QORA_HIP_MLP", "1")
    w = _model(pkg, seed=12)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    assert be.mlp_fused()
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    prompt = pkg.synth_tokens(12, 2700, 8, w.config.vocab)
    ref, _ = om.greedy(prompt, 24)
    _, first = be.raw_prefill(prompt, want_logits=False)
    assert [first] + be.generate_greedy(first, 23).tolist() == ref
