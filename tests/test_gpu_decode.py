"""Model-level parity on the GPU: raw_prefill / forward_decode_raw / greedy
decode through the C ABI against the oracle on the same seeded weights."""
import ctypes

import numpy as np
import pytest

import __graft_entry__ as entry
from helpers import REL_TOL, rel_err
from model_f64 import F64Model

pytestmark = pytest.mark.gpu


def small_model(pkg, fmt, layers=4, seed=0):
    cfg = entry.smoke_config(pkg)
    cfg.num_layers = layers
    return pkg.synthetic_model(cfg, seed=seed, fmt=fmt, rope_positions=128)


@pytest.mark.parametrize("fmt", [1, 0])
def test_prefill_decode_logits_and_kv_match_oracle(ctx, pkg, orc, fmt):
    w = small_model(pkg, fmt)
    prompt = pkg.synth_tokens(0, 2000, 13, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    truth = F64Model(w)
    logits, tok = be.raw_prefill(prompt)
    ref = om.prefill(prompt)
    assert rel_err(logits, ref) <= REL_TOL
    assert rel_err(logits, truth.prefill(prompt)) <= 1e-4
    assert tok == orc.argmax(ref)
    assert be.kv_len() == len(prompt)
    for layer in (0, 3):
        k, v = be.kv_layer(layer)
        kr, vr = om.kv_layer(layer)
        assert k.shape == kr.shape
        assert rel_err(k, kr) <= REL_TOL and rel_err(v, vr) <= REL_TOL
    # teacher-forced decode: feed fixed tokens, compare every step
    feed = pkg.synth_tokens(0, 2001, 20, w.config.vocab)
    for i, t in enumerate(feed):
        logits, tok = be.forward_decode_raw(int(t))
        ref = om.forward_decode(int(t))
        assert rel_err(logits, ref) <= REL_TOL
        if i % 5 == 0:
            assert rel_err(logits, truth.step(int(t))) <= 1e-4
        else:
            truth.step(int(t))
        gap = orc.top2_gap(ref)
        if gap > 1e-4 * float(np.max(np.abs(ref))):
            assert tok == orc.argmax(ref)
    assert be.kv_len() == len(prompt) + len(feed)


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_stale_nan_cache_slots_never_reach_the_output(ctx, pkg, orc, monkeypatch, kv_dtype):
    """The attention kernel reads cache slots at and past the appended
    position before they are written; they must be skipped, not multiplied
    by a zero weight (0 * NaN = NaN). The cache starts as NaN bit patterns."""
    monkeypatch.setenv("QORA_HIP_TUNING", "1")   # the library reads tuning variables only then
    monkeypatch.setenv("QORA_HIP_KV_FILL", "nan")
    w = small_model(pkg, 1)
    prompt = pkg.synth_tokens(0, 2000, 13, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128, kv_dtype=kv_dtype)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    logits, _ = be.raw_prefill(prompt)
    ref = om.prefill(prompt)
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    assert np.isfinite(logits).all()
    assert rel_err(logits, ref) <= tol
    for t in pkg.synth_tokens(0, 2001, 6, w.config.vocab):
        logits, _ = be.forward_decode_raw(int(t))
        ref = om.forward_decode(int(t))
        assert np.isfinite(logits).all()
        assert rel_err(logits, ref) <= tol


def test_greedy_tokens_match_oracle_small(ctx, pkg, orc):
    """64 greedy steps of an 8-layer model whose projection scales are x8, so
    that its greedy path visits many distinct tokens (48 of 64)."""
    w = small_model(pkg, 1, layers=8, seed=0)
    for ws in w.layers:
        for wt in ws:
            wt.scales = (wt.scales.view(np.float16).astype(np.float32) * np.float32(8)).astype(
                np.float16).view(np.uint16)
    prompt = pkg.synth_tokens(0, 2000, 16, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    ref, gaps = om.greedy(prompt, 64)
    assert len(set(ref)) >= 32
    got = pkg.generate_greedy_host(be, prompt, 64)
    assert got == ref
    # the device-chained loop produces the same sequence
    _, first = be.raw_prefill(prompt, want_logits=False)
    chained = be.generate_greedy(first, 63)
    assert [first] + chained.tolist() == ref


def test_f16_kv_cache_close_to_f32(ctx, pkg, orc):
    w = small_model(pkg, 1)
    prompt = pkg.synth_tokens(0, 2000, 30, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128, kv_dtype=pkg.KV_F16)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    logits, _ = be.raw_prefill(prompt)
    ref = om.prefill(prompt)
    # f16 K/V rounding (2^-11 relative) is the only difference from the f32 path
    assert rel_err(logits, ref) <= 5e-3


def test_state_errors(ctx, pkg):
    w = small_model(pkg, 1, layers=4)
    be = pkg.HipBackend(ctx, w, kv_capacity=8)
    with pytest.raises(pkg.QoraHipError) as e:
        be.forward_decode_raw(w.config.vocab)   # token out of range
    assert e.value.code == pkg.QORA_HIP_E_INVALID
    be.raw_prefill([1, 2, 3, 4, 5, 6, 7, 8])
    with pytest.raises(pkg.QoraHipError) as e:
        be.forward_decode_raw(1)               # cache full
    assert e.value.code == pkg.QORA_HIP_E_STATE
    be.kv_reset()
    assert be.kv_len() == 0
    be.forward_decode_raw(1)
    assert be.kv_len() == 1
    with pytest.raises(pkg.QoraHipError):
        be.raw_prefill([])


def test_qora_file_roundtrip_loads_same_model(ctx, pkg, tmp_path):
    w = small_model(pkg, 1)
    path = str(tmp_path / "m.qora")
    pkg.save_model(w, path)
    prompt = pkg.synth_tokens(0, 2000, 9, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    ref, _ = be.raw_prefill(prompt)
    ctx.check(ctx.lib.qora_hip_load_model(ctx.h, path.encode(), 64, 0), "load_model")
    logits = np.empty(w.config.vocab, dtype=np.float32)
    tok = ctypes.c_uint32()
    ids = np.asarray(prompt, dtype=np.uint32)
    ctx.check(ctx.lib.qora_hip_prefill(ctx.h, ids.ctypes.data, ids.size, logits.ctypes.data, ctypes.byref(tok)),
              "prefill")
    assert np.array_equal(logits, ref)


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_kv_upload_round_trip_is_bit_exact(ctx, pkg, kv_dtype):
    """kv_download -> kv_reset -> kv_upload restores the cache exactly: the next
    decode step gives the same logits, bit for bit, as without the round trip."""
    w = small_model(pkg, 1)
    L = w.config.num_layers
    prompt = pkg.synth_tokens(0, 2000, 21, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128, kv_dtype=kv_dtype)
    be.raw_prefill(prompt, want_logits=False)
    saved = [be.kv_layer(l) for l in range(L)]
    want, wtok = be.forward_decode_raw(77)
    be.kv_reset()
    for l, (k, v) in enumerate(saved):
        be.kv_upload(l, k, v)
    assert be.kv_len() == len(prompt)
    got, gtok = be.forward_decode_raw(77)
    assert np.array_equal(got, want) and gtok == wtok
    assert be.kv_len() == len(prompt) + 1


def test_kv_upload_rounds_to_f16_nearest_even(ctx, pkg):
    w = small_model(pkg, 1)
    kvd = w.config.num_kv_heads * w.config.head_dim
    be = pkg.HipBackend(ctx, w, kv_capacity=64, kv_dtype=pkg.KV_F16)
    r = np.random.default_rng(5)
    k = (r.standard_normal((40, kvd)) * np.exp2(r.integers(-20, 17, (40, kvd)))).astype(np.float32)
    k[0, :4] = [65519.0, 65520.0, -1e9, 2.0 ** -25]    # largest finite, overflow, underflow to zero
    v = r.standard_normal((40, kvd)).astype(np.float32)
    be.kv_upload(2, k, v)
    gk, gv = be.kv_layer(2)
    with np.errstate(over="ignore"):
        assert np.array_equal(gk, k.astype(np.float16).astype(np.float32))
    assert np.array_equal(gv, v.astype(np.float16).astype(np.float32))
    be.kv_upload(2, k[:0], v[:0])
    assert be.kv_len() == 0


def test_kv_upload_errors(ctx, pkg):
    w = small_model(pkg, 1)
    kvd = w.config.num_kv_heads * w.config.head_dim
    be = pkg.HipBackend(ctx, w, kv_capacity=16)
    z = np.zeros((17, kvd), np.float32)
    with pytest.raises(pkg.QoraHipError):
        be.kv_upload(0, z, z)                       # beyond the capacity
    with pytest.raises(pkg.QoraHipError):
        be.kv_upload(w.config.num_layers, z[:4], z[:4])
    with pytest.raises(pkg.QoraHipError):
        ctx.check(ctx.lib.qora_hip_kv_upload(ctx.h, 0, None, None, 3), "kv_upload")
    be.kv_upload(0, z[:16], z[:16])
    with pytest.raises(pkg.QoraHipError) as e:
        be.forward_decode_raw(1)                    # cache full
    assert e.value.code == pkg.QORA_HIP_E_STATE


@pytest.mark.parametrize("kv_dtype,hd,cap,n", [(0, 128, 8192, 6001), (1, 128, 8192, 6001), (1, 64, 8192, 6001),
                                               (1, 128, 16384, 9001), (1, 64, 16384, 9001)])
def test_long_context_decode_matches_oracle(ctx, pkg, orc, kv_dtype, hd, cap, n):
    """Decode over a cache of ~6000 uploaded positions (capacity 8192): the
    split length follows the context (96 positions per split here) and each
    attention block runs four subgroups; the appended row lands in a pass
    owned by a later subgroup (the direct kernel, for an f16 cache: a later
    wave), at capacities 8192 and 16384."""
    heads, kvh = (16, 4) if hd == 128 else (4, 2)
    cfg = pkg.ModelConfig(num_layers=4, vocab=1000, hidden=256, intermediate=704, num_heads=heads,
                          num_kv_heads=kvh, head_dim=hd, rope_half_dim=hd // 2, rope_theta=5e6, rope_positions=cap)
    w = pkg.synthetic_model(cfg, seed=4, rope_positions=cap)
    be = pkg.HipBackend(ctx, w, kv_capacity=cap, kv_dtype=kv_dtype)
    om = orc.OracleModel(w, kv_capacity=cap, T=4)
    r = np.random.default_rng(11)
    for layer in range(cfg.num_layers):
        k = r.standard_normal((n, kvh * hd), dtype=np.float32)
        v = r.standard_normal((n, kvh * hd), dtype=np.float32)
        if kv_dtype:
            k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
        be.kv_upload(layer, k, v)
        om.kv_set(layer, k, v)
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    for t in pkg.synth_tokens(4, 2001, 4, cfg.vocab):
        print(f"case long-context decode kv_dtype={kv_dtype} hd={hd} pos={be.kv_len()}", flush=True)
        logits, _ = be.forward_decode_raw(int(t))
        ref = om.forward_decode(int(t))
        assert rel_err(logits, ref) <= tol
    assert be.kv_len() == n + 4


@pytest.mark.parametrize("kv_dtype,n,cap", [(0, 2999, 8192), (1, 2999, 8192), (1, 4090, 8192), (0, 600, 8192),
                                             (1, 8180, 8192), (1, 8188, 16384), (0, 8188, 16384)])
def test_split_steps_below_4096_positions_at_a_large_capacity(ctx, pkg, orc, kv_dtype, n, cap):
    """A capacity of 8192 splits into 128-position pieces, so its split steps
    would run the long-context attention; steps that append a position below
    4096 run the one-subgroup split attention from their own graph instead
    (64-position splits past 2048: two passes a split). Logits against the
    oracle, the steps crossing from one graph to the other at 4096, and
    split steps near 8192 positions at capacities 8192 and 16384."""
    print(f"case split steps below 4096 kv_dtype={kv_dtype} n={n} cap={cap}", flush=True)
    cfg = pkg.ModelConfig(num_layers=3, vocab=1000, hidden=256, intermediate=704, num_heads=4,
                          num_kv_heads=2, head_dim=64, rope_half_dim=32, rope_theta=5e6, rope_positions=cap)
    w = pkg.synthetic_model(cfg, seed=12, rope_positions=cap)
    be = pkg.HipBackend(ctx, w, kv_capacity=cap, kv_dtype=kv_dtype)
    om = orc.OracleModel(w, kv_capacity=cap, T=4)
    r = np.random.default_rng(n)
    kvd = cfg.num_kv_heads * cfg.head_dim
    for layer in range(cfg.num_layers):
        k = r.standard_normal((n, kvd), dtype=np.float32) * np.linspace(0.5, 3, n, dtype=np.float32)[:, None]
        v = r.standard_normal((n, kvd), dtype=np.float32)
        if kv_dtype:
            k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
        be.kv_upload(layer, k, v)
        om.kv_set(layer, k, v)
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    for t in pkg.synth_tokens(12, 2001, 10, cfg.vocab):
        logits, _ = be.forward_decode_raw(int(t))
        assert rel_err(logits, om.forward_decode(int(t))) <= tol, (be.kv_len(), int(t))
    assert be.kv_len() == n + 10


@pytest.mark.parametrize("cap,n", [(2100, 1500), (3000, 2040), (2100, 2095)])
def test_split_count_covers_contexts_below_an_odd_capacity(ctx, pkg, orc, cap, n):
    """The split length follows the live context (32 positions up to 2048),
    so at a capacity whose own split length is longer (2100: 64 positions)
    a context of 1500 needs 47 splits where the capacity's geometry has 33:
    the step launches enough splits for every context up to the capacity,
    and no position goes unattended."""
    print(f"case split count cap={cap} n={n}", flush=True)
    cfg = pkg.ModelConfig(num_layers=2, vocab=1000, hidden=256, intermediate=704, num_heads=4,
                          num_kv_heads=2, head_dim=64, rope_half_dim=32, rope_theta=5e6, rope_positions=cap)
    w = pkg.synthetic_model(cfg, seed=8, rope_positions=cap)
    be = pkg.HipBackend(ctx, w, kv_capacity=cap)
    om = orc.OracleModel(w, kv_capacity=cap, T=4)
    r = np.random.default_rng(cap + n)
    kvd = cfg.num_kv_heads * cfg.head_dim
    for layer in range(cfg.num_layers):
        # keys that make the late positions matter: scores grow with position
        k = r.standard_normal((n, kvd), dtype=np.float32) * np.linspace(0.5, 3, n, dtype=np.float32)[:, None]
        v = r.standard_normal((n, kvd), dtype=np.float32)
        be.kv_upload(layer, k, v)
        om.kv_set(layer, k, v)
    for t in pkg.synth_tokens(8, 2001, 3, cfg.vocab):
        logits, _ = be.forward_decode_raw(int(t))
        assert rel_err(logits, om.forward_decode(int(t))) <= REL_TOL, int(t)


def test_state_calls_right_after_a_logits_free_step(ctx, pkg, orc):
    """A greedy step without logits returns once the device has stored its
    token, before the stream reports completion. Calls made right after it
    (cache read-back, reset, a new prompt) see the step's results complete."""
    print("case state calls after logits-free steps", flush=True)
    w = small_model(pkg, 1, layers=4, seed=9)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    prompt = pkg.synth_tokens(9, 2100, 12, w.config.vocab)
    ref, _ = om.greedy(prompt, 9)
    for _ in range(3):
        _, tok = be.raw_prefill(prompt, want_logits=False)
        got = [tok]
        for _ in range(8):
            _, tok = be.forward_decode_raw(int(tok), want_logits=False)
            got.append(tok)
            assert be.kv_len() == len(prompt) + len(got) - 1
        assert got == ref
        k, _ = be.kv_layer(2)
        assert k.shape[0] == len(prompt) + 8
        be.kv_reset()
        assert be.kv_len() == 0
    om2 = orc.OracleModel(w, kv_capacity=128, T=4)
    om2.prefill(prompt)
    for t in ref[:8]:
        om2.forward_decode(int(t))
    kr, _ = om2.kv_layer(2)
    assert rel_err(k, kr) <= REL_TOL


def test_model_reinit_right_after_a_logits_free_step(ctx, pkg, orc):
    """model_init right after a greedy step that returned without waiting for
    the stream: the old graphs and buffers are released only after the step
    has finished, and the new model runs correctly."""
    print("case model re-init after a logits-free step", flush=True)
    w = small_model(pkg, 1, layers=4, seed=10)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    prompt = pkg.synth_tokens(10, 2100, 12, w.config.vocab)
    _, tok = be.raw_prefill(prompt, want_logits=False)
    for _ in range(3):
        _, tok = be.forward_decode_raw(int(tok), want_logits=False)
    w2 = small_model(pkg, 1, layers=4, seed=11)
    be2 = pkg.HipBackend(ctx, w2, kv_capacity=128)
    om = orc.OracleModel(w2, kv_capacity=128, T=4)
    ref, _ = om.greedy(prompt, 5)
    got = pkg.generate_greedy_host(be2, prompt, 5)
    assert got == ref


def test_steps_refused_during_capture(ctx, pkg):
    """Decode, prefill and state calls read results back to the host: during a
    caller's stream capture they are refused (E_STATE) and the capture stays
    usable."""
    print("case steps refused during capture", flush=True)
    w = small_model(pkg, 1, layers=2, seed=12)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    prompt = pkg.synth_tokens(12, 2100, 5, w.config.vocab)
    _, tok = be.raw_prefill(prompt, want_logits=False)
    n0 = be.kv_len()
    out = ctypes.c_uint32()
    ids = np.asarray(prompt, dtype=np.uint32)
    ctx.capture_begin()
    try:
        assert ctx.lib.qora_hip_decode(ctx.h, int(tok), None, ctypes.byref(out)) == -4
        assert ctx.lib.qora_hip_prefill(ctx.h, ids.ctypes.data, ids.size, None, ctypes.byref(out)) == -4
        assert ctx.lib.qora_hip_kv_reset(ctx.h) == -4
    finally:
        g = ctx.capture_end()
        ctx.graph_destroy(g)
    assert be.kv_len() == n0
    _, nxt = be.forward_decode_raw(int(tok), want_logits=False)
    assert be.kv_len() == n0 + 1


@pytest.mark.parametrize("fmt", [1, 0])
def test_fixed_point_range_overflow_is_reported(ctx, pkg, fmt):
    """A down projection whose terms reach 2^20 would wrap the int64
    residual: the step returns QORA_HIP_E_RANGE instead of logits, and steps
    stay refused until the cache is reset."""
    print(f"case fixed-point range fmt={fmt}", flush=True)
    w = small_model(pkg, fmt, layers=2, seed=13)
    gate, up, down = w.layers[0][4:7]
    # gate == up, scaled by 100: every SwiGLU value silu(g) g = g^2 sigmoid(g)
    # is >= 0 and about half are ~1e3; down terms of 60000 then put each K
    # slice's sum far beyond 2^20, whatever the token
    if fmt == 1:
        gate.scales = (gate.scales.view(np.float16).astype(np.float32) * 100).astype(np.float16).view(np.uint16)
        up.packed, up.scales = gate.packed.copy(), gate.scales.copy()
        down.scales = np.full_like(down.scales, 0x7B53)          # 60000
    else:
        gate.data = (gate.data.view(np.float16).astype(np.float32) * 100).astype(np.float16).view(np.uint16)
        up.data = gate.data.copy()
        down.data = np.full_like(down.data, 0x7B53)
    prompt = pkg.synth_tokens(13, 2100, 6, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    be.raw_prefill(prompt, want_logits=False)                      # batched prefill: fp32, unguarded
    for want in (True, False, True):
        with pytest.raises(pkg.QoraHipError) as e:
            be.forward_decode_raw(3, want_logits=want)
        assert e.value.code == pkg.QORA_HIP_E_RANGE
    be.kv_reset()
    with pytest.raises(pkg.QoraHipError) as e:
        be.generate_greedy(3, 4)
    assert e.value.code == pkg.QORA_HIP_E_RANGE
    # the sampled step, with and without logits: the flag is reported there
    # too, and the next step is refused
    sp = pkg.SampleParams(temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.1, presence_penalty=0.0)
    for want in (False, True, False):
        be.kv_reset()
        be.raw_prefill(prompt, want_logits=False)
        with pytest.raises(pkg.QoraHipError) as e:
            be.decode_sample(3, list(prompt), sp, 12345, want_logits=want)
        assert e.value.code == pkg.QORA_HIP_E_RANGE
        with pytest.raises(pkg.QoraHipError) as e:
            be.decode_sample(3, list(prompt), sp, 12345, want_logits=False)
        assert e.value.code == pkg.QORA_HIP_E_RANGE
    # the same weights with the terms in range decode normally
    w2 = small_model(pkg, fmt, layers=2, seed=13)
    be2 = pkg.HipBackend(ctx, w2, kv_capacity=64)
    be2.raw_prefill(prompt, want_logits=False)
    be2.forward_decode_raw(3, want_logits=False)


def test_default_kv_capacity_is_the_rope_table(ctx, pkg, orc):
    """kv_capacity 0: the cache holds every position the RoPE tables cover (a
    caller never runs out where the reference's growing cache would go on);
    the step past the table is refused."""
    print("case default kv capacity", flush=True)
    w = small_model(pkg, 1, layers=4, seed=14)          # RoPE on layer 3, tables of 128 positions
    be = pkg.HipBackend(ctx, w, kv_capacity=0)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    prompt = pkg.synth_tokens(14, 2100, 100, w.config.vocab)
    _, tok = be.raw_prefill(prompt, want_logits=False)
    om.prefill(prompt)
    toks = be.generate_greedy(tok, 28)
    assert be.kv_len() == 128
    for t in [tok] + list(toks[:-1]):
        ref = om.forward_decode(int(t))
    assert int(toks[-1]) == orc.argmax(ref) or orc.top2_gap(ref) <= 1e-4 * float(np.max(np.abs(ref)))
    with pytest.raises(pkg.QoraHipError) as e:
        be.forward_decode_raw(int(toks[-1]))
    assert e.value.code == pkg.QORA_HIP_E_STATE


def test_forced_failures_leave_the_context_usable(ctx, pkg, orc, monkeypatch):
    """The reference sends any Err of the GPU backend to the CPU path
    (main.rs:143-151, gpu_inference.rs:518-562), so a failed call must come
    back as a clean error code and leave the context usable:
    QORA_HIP_FORCE_FAIL=alloc fails every device allocation (model set-up,
    the prefill's first buffers) and =launch every step before it launches.
    A refused step leaves the cache as it was, a refused prefill leaves it
    empty, a refused model_init leaves no model; the next call after the
    variable is cleared matches the oracle."""
    print("case forced alloc/launch failures", flush=True)
    w = small_model(pkg, 1, layers=4, seed=21)
    prompt = pkg.synth_tokens(21, 2000, 11, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    om = orc.OracleModel(w, kv_capacity=64, T=4)

    # alloc: the batched prefill's buffers are allocated by its first call
    monkeypatch.setenv("QORA_HIP_FORCE_FAIL", "alloc")
    with pytest.raises(pkg.QoraHipError) as e:
        be.raw_prefill(prompt)
    assert e.value.code == pkg.QORA_HIP_E_NOMEM
    assert be.kv_len() == 0
    monkeypatch.delenv("QORA_HIP_FORCE_FAIL")
    logits, tok = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= REL_TOL

    # launch: decode, device-chained greedy, sampled decode and prefill
    sp = pkg.SampleParams(**pkg.DEFAULT_SAMPLING)
    monkeypatch.setenv("QORA_HIP_FORCE_FAIL", "launch")
    for call in (lambda: be.forward_decode_raw(tok), lambda: be.forward_decode_raw(tok, want_logits=False),
                 lambda: be.generate_greedy(tok, 3), lambda: be.decode_sample(tok, list(prompt), sp, 99)):
        with pytest.raises(pkg.QoraHipError) as e:
            call()
        assert e.value.code == pkg.QORA_HIP_E_DEVICE
        assert be.kv_len() == len(prompt)
    monkeypatch.delenv("QORA_HIP_FORCE_FAIL")
    for t in (tok, 5, 17):
        logits, _ = be.forward_decode_raw(int(t))
        assert rel_err(logits, om.forward_decode(int(t))) <= REL_TOL
    monkeypatch.setenv("QORA_HIP_FORCE_FAIL", "launch")
    with pytest.raises(pkg.QoraHipError) as e:
        be.raw_prefill(prompt)
    assert e.value.code == pkg.QORA_HIP_E_DEVICE
    assert be.kv_len() == 0
    monkeypatch.delenv("QORA_HIP_FORCE_FAIL")
    om = orc.OracleModel(w, kv_capacity=64, T=4)
    logits, tok = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= REL_TOL

    # alloc during model_init: no model is left, steps are refused, and the
    # next model_init builds it again
    monkeypatch.setenv("QORA_HIP_FORCE_FAIL", "alloc")
    with pytest.raises(pkg.QoraHipError) as e:
        be.model_init()
    assert e.value.code == pkg.QORA_HIP_E_NOMEM
    monkeypatch.delenv("QORA_HIP_FORCE_FAIL")
    with pytest.raises(pkg.QoraHipError) as e:
        be.forward_decode_raw(tok)
    assert e.value.code == pkg.QORA_HIP_E_STATE
    be.model_init()
    om = orc.OracleModel(w, kv_capacity=64, T=4)
    logits, tok = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= REL_TOL
    logits, _ = be.forward_decode_raw(tok)
    assert rel_err(logits, om.forward_decode(tok)) <= REL_TOL


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_eager_launches_match_the_captured_graphs(ctx, pkg, monkeypatch, kv_dtype):
    """QORA_HIP_EAGER=1 launches a step kernel by kernel (for profilers that
    do not follow graphs): the same kernels and arguments as the graph the
    host picks for the step, so the logits are bit-identical. Steps from each
    attention variant of a capacity of 8192: fused (below 256 positions),
    chunked (below 512), one-subgroup split (below 4096), the long-context
    kernel above."""
    cap = 8192
    cfg = pkg.ModelConfig(num_layers=2, vocab=1000, hidden=256, intermediate=704, num_heads=4,
                          num_kv_heads=2, head_dim=64, rope_half_dim=32, rope_theta=5e6, rope_positions=cap)
    w = pkg.synthetic_model(cfg, seed=21, rope_positions=cap)
    be = pkg.HipBackend(ctx, w, kv_capacity=cap, kv_dtype=kv_dtype)
    kvd = cfg.num_kv_heads * cfg.head_dim
    toks = [int(t) for t in pkg.synth_tokens(21, 2001, 3, cfg.vocab)]
    for n in (100, 300, 3000, 5000, 8100):
        print(f"case eager vs graph kv_dtype={kv_dtype} n={n}", flush=True)
        r = np.random.default_rng(n)
        cache = [(r.standard_normal((n, kvd), dtype=np.float32), r.standard_normal((n, kvd), dtype=np.float32))
                 for _ in range(cfg.num_layers)]
        runs = []
        for eager in ("0", "1"):
            monkeypatch.setenv("QORA_HIP_EAGER", eager)
            for layer, (k, v) in enumerate(cache):
                be.kv_upload(layer, k, v)
            runs.append([be.forward_decode_raw(t)[0].copy() for t in toks])
            assert be.kv_len() == n + len(toks)
        for a, b in zip(*runs):
            assert np.array_equal(a, b), n
