"""The fused decode steps on the GPU: each layer's attention computed inside
the o-projection kernel (gemv_q4m_attn_kernel) for steps that append a
position below qora_hip_attn_o_limit (every workgroup over the whole
context), the chunked step up to qora_hip_attn_chunk_limit (each column-tile
workgroup of a head over its own chunk of positions, the chunk states
exchanged between the workgroups), and the split attention kernel above.
Against the oracle (gemv.rs:914-989 inside forward_decode_raw,
gemv.rs:872-1019), across the bounds, from the first position, at every
compiled pass count, and with f32 and f16 caches."""
import numpy as np
import pytest

import __graft_entry__ as entry
from helpers import REL_TOL, rel_err

pytestmark = pytest.mark.gpu


def _model(pkg, hd, layers=4, seed=0, positions=1024, fmt=1):
    if hd == 64:
        cfg = entry.smoke_config(pkg)
    else:
        cfg = pkg.ModelConfig(num_layers=layers, vocab=1000, hidden=256, intermediate=704, num_heads=16,
                              num_kv_heads=4, head_dim=128, rope_half_dim=64, rope_theta=5e6,
                              rope_positions=positions)
    cfg.num_layers = layers
    cfg.rope_positions = positions
    return pkg.synthetic_model(cfg, seed=seed, fmt=fmt, rope_positions=positions)


def test_limit_policy(ctx, pkg, monkeypatch):
    w = _model(pkg, 64)
    be = pkg.HipBackend(ctx, w, kv_capacity=512)
    assert be.attn_o_limit() == 256                       # the default bound
    be = pkg.HipBackend(ctx, w, kv_capacity=100)
    assert be.attn_o_limit() == 100                       # never above the capacity
    monkeypatch.setenv("QORA_HIP_ATTN_O", "0")
    assert pkg.HipBackend(ctx, w, kv_capacity=128).attn_o_limit() == 0
    monkeypatch.setenv("QORA_HIP_ATTN_O", "40")
    assert pkg.HipBackend(ctx, _model(pkg, 128), kv_capacity=128).attn_o_limit() == 40
    monkeypatch.setenv("QORA_HIP_ATTN_O", "640")                # the kernel takes at most 256 positions
    assert pkg.HipBackend(ctx, _model(pkg, 128), kv_capacity=1024).attn_o_limit() == 256
    monkeypatch.delenv("QORA_HIP_ATTN_O")
    # F16 weights run the VALU GEMVs: no fused step
    assert pkg.HipBackend(ctx, _model(pkg, 64, fmt=0), kv_capacity=128).attn_o_limit() == 0
    assert pkg.HipBackend(ctx, _model(pkg, 64, fmt=0), kv_capacity=128).attn_chunk_limit() == 0


def test_chunk_limit_policy(ctx, pkg, monkeypatch):
    """The chunked step covers [attn_o_limit, attn_chunk_limit): by default
    32 positions per column tile, at most 8 passes of 32 positions per tile,
    never above the capacity, and never at or below the fused bound;
    QORA_HIP_ATTN_CHUNK sets it."""
    w = _model(pkg, 128, positions=4096)
    monkeypatch.setenv("QORA_HIP_ATTN_CHUNK", "1000000")
    top = pkg.HipBackend(ctx, w, kv_capacity=4096).attn_chunk_limit()
    assert top > 256 and top % 256 == 0                 # 8 passes x 32 positions x the column tiles
    tiles = top // 256
    monkeypatch.delenv("QORA_HIP_ATTN_CHUNK")
    dflt = 32 * tiles if 32 * tiles > 256 else 0        # none when at or below the fused bound
    assert pkg.HipBackend(ctx, w, kv_capacity=4096).attn_chunk_limit() == dflt
    assert pkg.HipBackend(ctx, w, kv_capacity=300).attn_chunk_limit() == (300 if dflt else 0)
    assert pkg.HipBackend(ctx, w, kv_capacity=256).attn_chunk_limit() == 0   # all fused
    monkeypatch.setenv("QORA_HIP_ATTN_CHUNK", "0")
    assert pkg.HipBackend(ctx, w, kv_capacity=1024).attn_chunk_limit() == 0
    monkeypatch.setenv("QORA_HIP_ATTN_CHUNK", "600")
    assert pkg.HipBackend(ctx, w, kv_capacity=1024).attn_chunk_limit() == min(600, top)
    monkeypatch.setenv("QORA_HIP_ATTN_O", "0")          # chunked from the first position
    be = pkg.HipBackend(ctx, w, kv_capacity=1024)
    assert be.attn_o_limit() == 0 and be.attn_chunk_limit() == min(600, top)


@pytest.mark.parametrize("after", ["split", "chunked"])
@pytest.mark.parametrize("hd,kv_dtype", [(64, 0), (128, 0), (128, 1), (64, 1)])
def test_steps_across_the_bound_match_oracle(ctx, pkg, orc, monkeypatch, hd, kv_dtype, after):
    """Bound 24: a 12-token prompt, then 24 teacher-forced steps appending
    positions 12..35 (fused up to 23, split or chunked from 24 on)."""
    print(f"case attn_o across bound hd={hd} kv={kv_dtype} then {after}", flush=True)
    monkeypatch.setenv("QORA_HIP_ATTN_O", "24")
    if after == "split":
        monkeypatch.setenv("QORA_HIP_ATTN_CHUNK", "0")
    w = _model(pkg, hd, positions=128)
    be = pkg.HipBackend(ctx, w, kv_capacity=128, kv_dtype=kv_dtype)
    assert be.attn_o_limit() == 24
    assert (be.attn_chunk_limit() == 0) == (after == "split")
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    prompt = pkg.synth_tokens(hd, 2000, 12, w.config.vocab)
    logits, _ = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= tol
    for t in pkg.synth_tokens(hd, 2001, 24, w.config.vocab):
        pos = be.kv_len()
        logits, tok = be.forward_decode_raw(int(t))
        ref = om.forward_decode(int(t))
        assert rel_err(logits, ref) <= tol, pos
        if orc.top2_gap(ref) > 1e-4 * float(np.max(np.abs(ref))):
            assert tok == orc.argmax(ref), pos
    for layer in (0, w.config.num_layers - 1):
        k, v = be.kv_layer(layer)
        kr, vr = om.kv_layer(layer)
        assert rel_err(k, kr) <= tol and rel_err(v, vr) <= tol


@pytest.mark.parametrize("hd", [64, 128])
def test_fused_from_the_first_position(ctx, pkg, orc, monkeypatch, hd):
    """Token-by-token prefill: the first step appends position 0 with no
    cached row to read."""
    print(f"case attn_o first position hd={hd}", flush=True)
    monkeypatch.setenv("QORA_HIP_PREFILL", "seq")
    w = _model(pkg, hd, positions=64)
    be = pkg.HipBackend(ctx, w, kv_capacity=64)
    assert be.attn_o_limit() == 64
    om = orc.OracleModel(w, kv_capacity=64, T=4)
    for n in (1, 5):
        be.kv_reset()
        prompt = pkg.synth_tokens(hd + n, 2100, n, w.config.vocab)
        logits, _ = be.raw_prefill(prompt)
        assert rel_err(logits, om.prefill(prompt)) <= REL_TOL, n
    k, v = be.kv_layer(1)
    kr, vr = om.kv_layer(1)
    assert rel_err(k, kr) <= REL_TOL and rel_err(v, vr) <= REL_TOL


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_fused_every_pass_count(ctx, pkg, orc, kv_dtype):
    """The fused kernel is compiled per count of 32-position passes (1..8).
    Caches of n uploaded positions, then two steps appending n and n + 1,
    for n around every pass boundary: each pass count, the appended row as
    the first, a middle and the last position of its pass, and the step from
    the last fused position (255) to the step kind above the bound (256)."""
    print(f"case attn_o pass counts kv={kv_dtype}", flush=True)
    cap = 320
    w = _model(pkg, 128, positions=cap, seed=5)
    be = pkg.HipBackend(ctx, w, kv_capacity=cap, kv_dtype=kv_dtype)
    assert be.attn_o_limit() == 256
    om = orc.OracleModel(w, kv_capacity=cap, T=4)
    r = np.random.default_rng(21)
    kvd = w.config.num_kv_heads * w.config.head_dim
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    for n in (0, 1, 30, 31, 32, 45, 63, 64, 95, 96, 127, 150, 159, 191, 192, 223, 224, 240, 254, 255):
        for layer in range(w.config.num_layers):
            k = r.standard_normal((n, kvd), dtype=np.float32)
            v = r.standard_normal((n, kvd), dtype=np.float32)
            if kv_dtype:
                k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
            be.kv_upload(layer, k, v)
            om.kv_set(layer, k, v)
        for t in pkg.synth_tokens(5, 2001 + n, 2, w.config.vocab):
            logits, _ = be.forward_decode_raw(int(t))
            assert rel_err(logits, om.forward_decode(int(t))) <= tol, n
        k, v = be.kv_layer(2)
        kr, vr = om.kv_layer(2)
        assert rel_err(k, kr) <= tol and rel_err(v, vr) <= tol, n


@pytest.mark.parametrize("bound,prompt_len,chunk", [(30, 10, "0"), (30, 10, None), (256, 25, None), (0, 40, None)])
def test_device_chained_greedy_crosses_the_bound(ctx, pkg, orc, monkeypatch, bound, prompt_len, chunk):
    """generate_greedy launches every step from the host in one call; each
    picks its graph by the position it appends: across the fused/split and
    fused/chunked bounds (30), across the fused kernel's pass counts
    (positions 25..64), and across the chunked step's (bound 0: chunked from
    the prompt, positions 40..79)."""
    monkeypatch.setenv("QORA_HIP_ATTN_O", str(bound))
    if chunk is not None:
        monkeypatch.setenv("QORA_HIP_ATTN_CHUNK", chunk)
    w = _model(pkg, 128, positions=128, seed=6)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    prompt = pkg.synth_tokens(6, 2000, prompt_len, w.config.vocab)
    ref, _ = om.greedy(prompt, 40)
    _, first = be.raw_prefill(prompt, want_logits=False)
    assert [first] + be.generate_greedy(first, 39).tolist() == ref


@pytest.mark.parametrize("mode,kv_dtype", [("chunked", 0), ("chunked", 1), ("split", 0)])
def test_chunked_every_pass_count(ctx, pkg, orc, monkeypatch, mode, kv_dtype):
    """The chunked step is compiled per count of 32-position passes per
    column tile (1..8); with the fused step off it runs from the first
    position. Caches of n uploaded positions, then two steps appending n and
    n + 1, for n around every chunk and pass-count boundary of the model's
    column tiles (chunks wholly past the context, the appended row as the
    first and last position of a chunk, the last position below the bound);
    the same positions through the split attention kernel (mode split)."""
    print(f"case chunked pass counts {mode} kv={kv_dtype}", flush=True)
    monkeypatch.setenv("QORA_HIP_ATTN_O", "0")
    monkeypatch.setenv("QORA_HIP_ATTN_CHUNK", "0" if mode == "split" else "1000000")
    w = _model(pkg, 128, positions=4096, seed=7)
    probe = pkg.HipBackend(ctx, w, kv_capacity=4096)
    top = probe.attn_chunk_limit()
    del probe
    if mode == "split":
        assert top == 0
        top = 512
    cap = top
    tiles = top // 256                                   # chunk of np passes: 32 np positions per column tile
    be = pkg.HipBackend(ctx, w, kv_capacity=cap, kv_dtype=kv_dtype)
    assert be.attn_o_limit() == 0
    assert be.attn_chunk_limit() == (cap if mode == "chunked" else 0)
    om = orc.OracleModel(w, kv_capacity=cap, T=4)
    r = np.random.default_rng(22)
    kvd = w.config.num_kv_heads * w.config.head_dim
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    step = 32 * tiles                                    # positions per pass count
    ns = {0, 1, 31, 32, 33, 63, 64, step - 2, step - 1, step, step + 1, 2 * step - 1, 2 * step + 31,
          3 * step + 64, 4 * step - 1, 5 * step + 7, 6 * step - 32, 7 * step, 8 * step - 3, cap - 2}
    for n in sorted(x for x in ns if 0 <= x <= cap - 2):
        for layer in range(w.config.num_layers):
            k = r.standard_normal((n, kvd), dtype=np.float32)
            v = r.standard_normal((n, kvd), dtype=np.float32)
            if kv_dtype:
                k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
            be.kv_upload(layer, k, v)
            om.kv_set(layer, k, v)
        for t in pkg.synth_tokens(7, 3001 + n, 2, w.config.vocab):
            logits, _ = be.forward_decode_raw(int(t))
            assert rel_err(logits, om.forward_decode(int(t))) <= tol, n
        k, v = be.kv_layer(3)
        kr, vr = om.kv_layer(3)
        assert rel_err(k, kr) <= tol and rel_err(v, vr) <= tol, n


def test_chunked_wait_timeout_is_reported(ctx, pkg, orc, monkeypatch):
    """The chunked step's workgroups wait a bounded number of polls for their
    head's chunk states; one that gives up flags the step, which then
    returns QORA_HIP_E_RANGE instead of results, and later steps are refused
    until the cache is reset. Forced from the host with a spin limit of 0
    (every workgroup gives up at once; all its accesses stay in bounds), then
    the same model with the normal limit decodes as the oracle does."""
    print("case chunked wait timeout", flush=True)
    monkeypatch.setenv("QORA_HIP_ATTN_O", "0")
    monkeypatch.setenv("QORA_HIP_ATTN_CHUNK", "1000000")
    monkeypatch.setenv("QORA_HIP_TUNING", "1")
    monkeypatch.setenv("QORA_HIP_CHUNK_SPIN", "0")
    w = _model(pkg, 128, positions=256, seed=8)
    prompt = pkg.synth_tokens(8, 2200, 20, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=256)
    assert be.attn_chunk_limit() > 0
    be.raw_prefill(prompt, want_logits=False)                # batched prefill: no chunked step
    for want in (True, False):
        with pytest.raises(pkg.QoraHipError) as e:
            be.forward_decode_raw(5, want_logits=want)
        assert e.value.code == pkg.QORA_HIP_E_RANGE
    monkeypatch.delenv("QORA_HIP_CHUNK_SPIN")
    be = pkg.HipBackend(ctx, w, kv_capacity=256)
    om = orc.OracleModel(w, kv_capacity=256, T=4)
    logits, _ = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= REL_TOL
    for t in (5, 9):
        logits, _ = be.forward_decode_raw(t)
        assert rel_err(logits, om.forward_decode(t)) <= REL_TOL
