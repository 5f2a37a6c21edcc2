"""The long-context plus prefill workload at model size, on the GPU against
the oracle: the 36-layer SmolLM3-3B architecture with seeded random Q4
weights (seed 1), a batched prefill of 512 seeded random token ids
(raw_prefill, gemv.rs:1027-1190), then decode steps with every layer's
binary16 KV cache filled to 32,700 positions (forward_decode_raw,
gemv.rs:872-1019), and decode steps over an f32 cache filled to 1990
positions (the 2048-context workload's split attention).

The filled cache rows are seeded N(0, 1) values rounded to binary16 (one
pool of rows, each layer's window starting one row further on) and set in
both the device cache (qora_hip_kv_upload) and the oracle's f32 cache
(oq_kv_set), so both attend over identical keys and values. The rows each
step appends are rounded to binary16 on the device only; the 5e-3 bound
covers that rounding (2^-11 relative per value). Greedy tokens are compared
wherever the oracle's top-2 logit gap exceeds 1e-4 (f32 cache) or twice the
bound times the largest logit (binary16 cache), so that the bound decides
the order."""
import time

import numpy as np
import pytest

from helpers import REL_TOL, rel_err

pytestmark = pytest.mark.gpu

N_PROMPT = 512
FILL = 32700
CAP = 32768
THREADS = 16
F16_TOL = 5e-3


@pytest.fixture(scope="module")
def model(pkg):
    return pkg.synthetic_model(pkg.SMOLLM3_3B, seed=1, rope_positions=CAP)


def test_prefill_512_matches_oracle(pkg, orc, model):
    print("case prefill 512 SmolLM3-3B seed 1", flush=True)
    c = model.config
    ids = pkg.synth_tokens(1, 2500, N_PROMPT, c.vocab)
    ctx = pkg.HipContext(0)
    try:
        be = pkg.HipBackend(ctx, model, kv_capacity=N_PROMPT + 8, kv_dtype=pkg.KV_F32)
        logits, tok = be.raw_prefill(ids)
        kv = {l: be.kv_layer(l) for l in (0, c.num_layers - 1)}
        # the same prompt into a binary16 cache
        be16 = pkg.HipBackend(ctx, model, kv_capacity=N_PROMPT + 8, kv_dtype=pkg.KV_F16)
        logits16, tok16 = be16.raw_prefill(ids)
        kv16 = be16.kv_layer(c.num_layers - 1)
    finally:
        ctx.close()
    orc.set_threads(THREADS)
    om = orc.OracleModel(model, kv_capacity=N_PROMPT + 8, T=THREADS)
    ref = om.prefill(ids)
    assert rel_err(logits, ref) <= REL_TOL
    for l, (k, v) in kv.items():
        kr, vr = om.kv_layer(l)
        assert k.shape == kr.shape == (N_PROMPT, c.num_kv_heads * c.head_dim)
        assert rel_err(k, kr) <= REL_TOL and rel_err(v, vr) <= REL_TOL, l
    assert rel_err(logits16, ref) <= F16_TOL
    kr, vr = om.kv_layer(c.num_layers - 1)
    assert rel_err(kv16[0], kr) <= REL_TOL and rel_err(kv16[1], vr) <= REL_TOL
    if orc.top2_gap(ref) > 1e-4:
        assert tok == orc.argmax(ref)
    if orc.top2_gap(ref) > 2 * F16_TOL * np.max(np.abs(ref)):
        assert tok16 == orc.argmax(ref)


def test_decode_over_32700_positions_f16_cache_matches_oracle(pkg, orc, model):
    print("case decode at 32700 positions, f16 KV, SmolLM3-3B seed 1", flush=True)
    c = model.config
    kvd = c.num_kv_heads * c.head_dim
    t0 = time.perf_counter()

    def phase(what):
        print(f"  {what}: {time.perf_counter() - t0:.1f} s", flush=True)

    orc.set_threads(THREADS)
    om = orc.OracleModel(model, kv_capacity=CAP, T=THREADS)
    ctx = pkg.HipContext(0)
    try:
        be = pkg.HipBackend(ctx, model, kv_capacity=CAP, kv_dtype=pkg.KV_F16)
        phase("model on device")
        # one seeded pool of rows; layer l's cache is pool rows l .. l + FILL - 1
        pool = np.random.default_rng(FILL).standard_normal((2, FILL + c.num_layers, kvd), dtype=np.float32)
        pool = pool.astype(np.float16).astype(np.float32)
        for layer in range(c.num_layers):
            k, v = pool[0, layer:layer + FILL], pool[1, layer:layer + FILL]
            be.kv_upload(layer, k, v)
            om.kv_set(layer, k, v)
        del pool, k, v
        phase("caches filled")
        assert be.kv_len() == FILL
        steps = pkg.synth_tokens(1, 2501, 3, c.vocab)
        for t in steps:
            logits, tok = be.forward_decode_raw(int(t))
            ref = om.forward_decode(int(t))
            phase(f"step {int(t)}")
            assert rel_err(logits, ref) <= F16_TOL, int(t)
            if orc.top2_gap(ref) > 2 * F16_TOL * np.max(np.abs(ref)):
                assert tok == orc.argmax(ref)
        assert be.kv_len() == FILL + len(steps)
        for l in (0, c.num_layers - 1):
            k, v = be.kv_layer(l)
            kr, vr = om.kv_layer(l)
            assert np.array_equal(k[:FILL], kr[:FILL]) and np.array_equal(v[:FILL], vr[:FILL]), l
            assert rel_err(k[FILL:], kr[FILL:]) <= REL_TOL and rel_err(v[FILL:], vr[FILL:]) <= REL_TOL, l
    finally:
        ctx.close()


def test_decode_over_1990_positions_f32_cache_matches_oracle(pkg, orc, model):
    """The 2048-context workload's decode path at model size: every layer's
    f32 cache filled to 1990 positions (the split attention past 256
    positions, 63 splits of 32), then 6 decode steps against the oracle at
    REL_TOL, logits and the appended cache rows; greedy tokens compared
    wherever the oracle's top-2 gap exceeds 1e-4 of its largest logit."""
    print("case decode at 1990 positions, f32 KV, SmolLM3-3B seed 1", flush=True)
    c = model.config
    kvd = c.num_kv_heads * c.head_dim
    fill, cap = 1990, 2048
    orc.set_threads(THREADS)
    om = orc.OracleModel(model, kv_capacity=cap, T=THREADS)
    ctx = pkg.HipContext(0)
    try:
        be = pkg.HipBackend(ctx, model, kv_capacity=cap, kv_dtype=pkg.KV_F32)
        pool = np.random.default_rng(fill).standard_normal((2, fill + c.num_layers, kvd), dtype=np.float32)
        for layer in range(c.num_layers):
            k, v = pool[0, layer:layer + fill], pool[1, layer:layer + fill]
            be.kv_upload(layer, k, v)
            om.kv_set(layer, k, v)
        del pool
        assert be.kv_len() == fill
        compared = 0
        for t in pkg.synth_tokens(1, 2502, 6, c.vocab):
            logits, tok = be.forward_decode_raw(int(t))
            ref = om.forward_decode(int(t))
            err = rel_err(logits, ref)
            print(f"  step token {int(t)}: rel err {err:.2e}", flush=True)
            assert err <= REL_TOL, int(t)
            if orc.top2_gap(ref) > 1e-4 * np.max(np.abs(ref)):
                assert tok == orc.argmax(ref)
                compared += 1
        assert compared >= 3
        for l in (0, 17, c.num_layers - 1):
            k, v = be.kv_layer(l)
            kr, vr = om.kv_layer(l)
            assert np.array_equal(k[:fill], kr[:fill]) and np.array_equal(v[:fill], vr[:fill]), l
            assert rel_err(k[fill:], kr[fill:]) <= REL_TOL and rel_err(v[fill:], vr[fill:]) <= REL_TOL, l
    finally:
        ctx.close()
