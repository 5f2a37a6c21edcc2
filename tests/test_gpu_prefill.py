"""Batched prefill on the GPU: the matrix-core GEMM (qora_hip_gemm), the
causal prefill attention (qora_hip_attn_prefill) and raw_prefill through the
model (qora_hip_prefill), against the oracle on the same seeded inputs.

The reference's gemm_q4 computes each row as gemv_q4_inner over the full k
(gemv.rs:680-706), which the oracle's gemv with T = 1 restates; the causal
attention row t equals the decode attention with L = pos0 + t + 1
(gemv.rs:1088-1130 vs 914-989)."""
import numpy as np
import pytest

import __graft_entry__ as entry
from helpers import REL_TOL, dequant_np, device, elem_err, exact_q4, rel_err, rng
from model_f64 import F64Model

pytestmark = pytest.mark.gpu

# Products are exact (binary16 parts of x and w, fp32 MFMA accumulation): the
# only difference from float64 is fp32 summation and the 22-bit split of x.
TRUTH_TOL = 1e-5


def _gemm(ctx, d, wid, x, T, n):
    y = d.empty(T * n * 4)
    ctx.check(ctx.lib.qora_hip_gemm(ctx.h, wid, d.put(x.astype(np.float32)), y, T, None), "gemm")
    return d.get(y, (T, n), np.float32)


@pytest.mark.parametrize("k,n,T", [(2048, 2048, 64), (2048, 512, 100), (11008, 2048, 65), (2048, 11008, 130),
                                   (256, 96, 1), (64, 32, 3), (128, 4096, 300)])
def test_gemm_q4_vs_oracle_and_truth(ctx, orc, pkg, k, n, T):
    print(f"case gemm q4 k={k} n={n} T={T}", flush=True)
    packed, scales = pkg.synth_q4(31, k + n, k, n)
    x = (rng(T + k).standard_normal((T, k)) * 3).astype(np.float32)
    wid = ctx.upload(pkg.Weight(k=k, n=n, packed=packed, scales=scales))
    with device(ctx) as d:
        y = _gemm(ctx, d, wid, x, T, n)
    W = dequant_np(packed, scales, k, n)
    truth = x.astype(np.float64) @ W
    assert rel_err(y, truth) <= TRUTH_TOL
    assert elem_err(y, truth, np.abs(x.astype(np.float64)) @ np.abs(W)) <= TRUTH_TOL
    for t in sorted({0, T // 2, T - 1}):
        ref = orc.gemv_q4(x[t], packed, scales, k, n, T=1)
        assert rel_err(y[t], ref) <= REL_TOL


@pytest.mark.parametrize("k,n,T", [(2048, 2048, 70), (512, 352, 5)])
def test_gemm_f16_vs_oracle_and_truth(ctx, orc, pkg, k, n, T):
    print(f"case gemm f16 k={k} n={n} T={T}", flush=True)
    w = pkg.synth_f16(32, k + n, k * n, 0.02)
    x = rng(T).standard_normal((T, k)).astype(np.float32)
    wid = ctx.upload(pkg.Weight(k=k, n=n, data=w))
    with device(ctx) as d:
        y = _gemm(ctx, d, wid, x, T, n)
    W = w.view(np.float16).astype(np.float64).reshape(k, n)
    truth = x.astype(np.float64) @ W
    assert rel_err(y, truth) <= TRUTH_TOL
    assert elem_err(y, truth, np.abs(x.astype(np.float64)) @ np.abs(W)) <= TRUTH_TOL
    for t in (0, T - 1):
        assert rel_err(y[t], orc.gemv_f16(x[t], w, k, n, T=1)) <= REL_TOL


@pytest.mark.parametrize("k,n,T", [(2048, 1024, 64), (4096, 256, 7)])
def test_gemm_exact_regime_bit_exact(ctx, pkg, k, n, T):
    """Power-of-two scales and small-integer x: every partial sum is an exact
    fp32 value, so any summation order gives the float64 result bit for bit."""
    r = rng(k * 3 + n)
    packed, scales = exact_q4(r, k, n)
    x = r.integers(-4, 5, size=(T, k)).astype(np.float32)
    wid = ctx.upload(pkg.Weight(k=k, n=n, packed=packed, scales=scales))
    with device(ctx) as d:
        y = _gemm(ctx, d, wid, x, T, n)
    truth = x.astype(np.float64) @ dequant_np(packed, scales, k, n)
    assert np.array_equal(y, truth.astype(np.float32))


def test_gemm_one_hot_rows_and_scale_extremes(ctx, pkg):
    """x = e_i gives row i of W exactly, also with the largest finite scale and
    a zero scale. A column group spanning 2^40 (65504 next to the smallest
    subnormal) keeps the small row to within 2^-39 of the group's largest
    value, not exactly: w' shares one power-of-two scale per group."""
    k, n = 256, 64
    r = rng(5)
    q = r.integers(0, 16, size=(k, n), dtype=np.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    s = np.abs(r.normal(0, 0.02, size=(k, n // 32))).astype(np.float16)
    s[3, 0] = np.float16(65504.0)
    s[4, 0] = np.float16(2.0 ** -24)
    s[5, 1] = np.float16(0.0)
    scales = s.view(np.uint16).reshape(-1)
    wid = ctx.upload(pkg.Weight(k=k, n=n, packed=packed, scales=scales))
    rows = [0, 3, 4, 5, 255]
    x = np.zeros((len(rows), k), np.float32)
    for i, rr in enumerate(rows):
        x[i, rr] = 1.0
    with device(ctx) as d:
        y = _gemm(ctx, d, wid, x, len(rows), n)
    W = dequant_np(packed, scales, k, n)
    for i, rr in enumerate(rows):
        if rr == 4:
            # half a binary16 subnormal step of w' (2^-25) times 2^f_g
            assert np.max(np.abs(y[i] - W[rr])) <= 2.0 ** -39 * np.max(np.abs(W[:, :32]))
            assert np.array_equal(y[i, 32:], W[rr, 32:].astype(np.float32))
        else:
            assert np.array_equal(y[i], W[rr].astype(np.float32)), rr


def test_gemm_errors(ctx, pkg):
    p, s = pkg.synth_q4(33, 1, 48, 64)
    wid = ctx.upload(pkg.Weight(k=48, n=64, packed=p, scales=s))   # k not a multiple of 32
    with device(ctx) as d:
        x = d.put(np.zeros((2, 48), np.float32))
        with pytest.raises(pkg.QoraHipError):
            ctx.check(ctx.lib.qora_hip_gemm(ctx.h, wid, x, d.empty(2 * 64 * 4), 2, None), "gemm")
        with pytest.raises(pkg.QoraHipError):
            ctx.check(ctx.lib.qora_hip_gemm(ctx.h, 10 ** 6, x, d.empty(16), 1, None), "gemm")


@pytest.mark.parametrize("pos0,T,hd,kv_f16", [(0, 1, 128, 0), (0, 37, 128, 0), (100, 64, 128, 1), (0, 200, 64, 0),
                                              (31, 33, 128, 1)])
def test_attn_prefill_vs_oracle(ctx, orc, pos0, T, hd, kv_f16):
    print(f"case attn_prefill pos0={pos0} T={T} hd={hd} f16={kv_f16}", flush=True)
    H, KVH = (16, 4) if hd == 128 else (4, 2)
    r = rng(pos0 * 7 + T)
    L = pos0 + T
    q = r.standard_normal((T, H * hd)).astype(np.float32)
    kc = r.standard_normal((L, KVH * hd)).astype(np.float32)
    vc = r.standard_normal((L, KVH * hd)).astype(np.float32)
    if kv_f16:
        kd, vd = kc.astype(np.float16), vc.astype(np.float16)
        kc, vc = kd.astype(np.float32), vd.astype(np.float32)
        kdev, vdev = kd.view(np.uint16), vd.view(np.uint16)
    else:
        kdev, vdev = kc, vc
    with device(ctx) as d:
        out = d.empty(T * H * hd * 4)
        ctx.check(ctx.lib.qora_hip_attn_prefill(ctx.h, d.put(q), d.put(kdev), d.put(vdev), kv_f16, pos0, T, H, KVH,
                                                hd, out, None), "attn_prefill")
        got = d.get(out, (T, H * hd), np.float32)
    for t in sorted({0, T // 3, T - 1}):
        n = pos0 + t + 1
        ref = orc.attention_decode(q[t], kc[:n].reshape(-1), vc[:n].reshape(-1), n, H, KVH, hd)
        assert rel_err(got[t], ref) <= REL_TOL, t


def _model(pkg, fmt, layers=4, seed=0, positions=128):
    cfg = entry.smoke_config(pkg)
    cfg.num_layers = layers
    cfg.rope_positions = positions
    return pkg.synthetic_model(cfg, seed=seed, fmt=fmt, rope_positions=positions)


@pytest.mark.parametrize("fmt,kv_dtype,n", [(1, 0, 2), (1, 0, 33), (1, 1, 100), (0, 0, 70)])
def test_batched_prefill_matches_oracle(ctx, pkg, orc, fmt, kv_dtype, n):
    print(f"case batched prefill fmt={fmt} kv={kv_dtype} n={n}", flush=True)
    w = _model(pkg, fmt)
    prompt = pkg.synth_tokens(0, 2100 + n, n, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128, kv_dtype=kv_dtype)
    om = orc.OracleModel(w, kv_capacity=128, T=4)
    logits, tok = be.raw_prefill(prompt)
    ref = om.prefill(prompt)
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    assert rel_err(logits, ref) <= tol
    if kv_dtype == 0:
        assert rel_err(logits, F64Model(w).prefill(prompt)) <= 1e-4
    if orc.top2_gap(ref) > 1e-4 * float(np.max(np.abs(ref))):
        assert tok == orc.argmax(ref)
    assert be.kv_len() == n
    for layer in (0, w.config.num_layers - 1):
        k, v = be.kv_layer(layer)
        kr, vr = om.kv_layer(layer)
        assert rel_err(k, kr) <= tol and rel_err(v, vr) <= tol
    for t in pkg.synth_tokens(0, 2200, 5, w.config.vocab):
        logits, _ = be.forward_decode_raw(int(t))
        assert rel_err(logits, om.forward_decode(int(t))) <= tol


def test_batched_prefill_in_chunks(ctx, pkg, orc):
    """600 tokens: two chunks of up to 512, the second attending to the first's
    cache rows."""
    w = _model(pkg, 1, layers=2, seed=2, positions=1024)
    prompt = pkg.synth_tokens(2, 2300, 600, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=1024)
    om = orc.OracleModel(w, kv_capacity=1024, T=8)
    logits, _ = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= REL_TOL
    k, v = be.kv_layer(1)
    kr, vr = om.kv_layer(1)
    assert k.shape == kr.shape == (600, w.config.num_kv_heads * w.config.head_dim)
    assert rel_err(k, kr) <= REL_TOL and rel_err(v, vr) <= REL_TOL


def test_batched_and_sequential_prefill_agree(ctx, pkg, orc, monkeypatch):
    w = _model(pkg, 1, layers=4, seed=3)
    prompt = pkg.synth_tokens(3, 2400, 40, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    batched, tb = be.raw_prefill(prompt)
    monkeypatch.setenv("QORA_HIP_PREFILL", "seq")
    seq, ts = be.raw_prefill(prompt)
    assert rel_err(batched, seq) <= REL_TOL
    if orc.top2_gap(seq) > 1e-4 * float(np.max(np.abs(seq))):
        assert tb == ts


@pytest.mark.parametrize("k,n,T", [(2048, 11008, 130), (2048, 512, 64)])
def test_gemm_loop_modes_bit_identical(ctx, pkg, monkeypatch, k, n, T):
    """The single-buffered K loop (default) and the double-buffered one
    (QORA_HIP_PF_MODE=0) issue the same products in the same order."""
    print(f"case gemm modes k={k} n={n} T={T}", flush=True)
    packed, scales = pkg.synth_q4(34, k + n, k, n)
    x = (rng(T + 3).standard_normal((T, k)) * 2).astype(np.float32)
    wid = ctx.upload(pkg.Weight(k=k, n=n, packed=packed, scales=scales))
    with device(ctx) as d:
        y1 = _gemm(ctx, d, wid, x, T, n)
        monkeypatch.setenv("QORA_HIP_TUNING", "1")   # the library reads tuning variables only then
        monkeypatch.setenv("QORA_HIP_PF_MODE", "0")
        y0 = _gemm(ctx, d, wid, x, T, n)
    assert np.array_equal(y0, y1)


@pytest.mark.parametrize("k,n,T", [(2048, 3072, 200), (11008, 2048, 77), (512, 1024, 33)])
def test_gemm2_tile_heights_bit_identical(ctx, pkg, monkeypatch, k, n, T):
    """32- and 64-token tiles of the packed-weight GEMM issue the same products
    per output element in the same order (K unsplit in both)."""
    print(f"case gemm2 tile heights k={k} n={n} T={T}", flush=True)
    packed, scales = pkg.synth_q4(36, k + n, k, n)
    x = (rng(T + 5).standard_normal((T, k)) * 2).astype(np.float32)
    wid = ctx.upload(pkg.Weight(k=k, n=n, packed=packed, scales=scales))
    monkeypatch.setenv("QORA_HIP_TUNING", "1")   # the library reads tuning variables only then
    monkeypatch.setenv("QORA_HIP_PF_SPLITS", "1")
    with device(ctx) as d:
        monkeypatch.setenv("QORA_HIP_PF_BM", "64")
        y64 = _gemm(ctx, d, wid, x, T, n)
        monkeypatch.setenv("QORA_HIP_PF_BM", "32")
        y32 = _gemm(ctx, d, wid, x, T, n)
    assert np.array_equal(y32, y64)
    W = dequant_np(packed, scales, k, n)
    assert rel_err(y32, x.astype(np.float64) @ W) <= TRUTH_TOL


@pytest.mark.parametrize("hidden,inter,heads", [(2048, 11008, 16), (512, 3008, 4)])
def test_row_producers_register_and_loop_bit_identical(ctx, pkg, monkeypatch, hidden, inter, heads):
    """The register-cached row producers (rows up to 2048, 4096 and 12288 wide)
    and the multi-pass ones (QORA_HIP_PF_ROWS=loop) compute the same values."""
    print(f"case row producers hidden={hidden} inter={inter}", flush=True)
    cfg = pkg.ModelConfig(num_layers=2, vocab=1000, hidden=hidden, intermediate=inter, num_heads=heads,
                          num_kv_heads=4, head_dim=128, rope_half_dim=64, rope_theta=5e6, rope_positions=128)
    w = pkg.synthetic_model(cfg, seed=9, fmt=1, rope_positions=128)
    prompt = pkg.synth_tokens(9, 2500, 70, cfg.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=128)
    reg, treg = be.raw_prefill(prompt)
    kreg, vreg = be.kv_layer(1)
    be.kv_reset()
    monkeypatch.setenv("QORA_HIP_TUNING", "1")   # the library reads tuning variables only then
    monkeypatch.setenv("QORA_HIP_PF_ROWS", "loop")
    loop, tloop = be.raw_prefill(prompt)
    kl, vl = be.kv_layer(1)
    assert np.array_equal(reg, loop) and treg == tloop
    assert np.array_equal(kreg, kl) and np.array_equal(vreg, vl)


@pytest.mark.parametrize("hd,kv_dtype,n,ch", [(64, 0, 150, "64"), (64, 1, 150, "64"), (128, 0, 200, "64"),
                                               (128, 1, 130, ""), (128, 0, 256, "")])
def test_batched_prefill_attention_key_chunks(ctx, pkg, orc, monkeypatch, hd, kv_dtype, n, ch):
    """The prefill attention with each query block's keys split into chunks
    (QORA_HIP_PF_ATTN_CH=64, else the default of 128 keys) and merged: logits,
    cache and the next decode step against the oracle."""
    print(f"case prefill key chunks hd={hd} kv={kv_dtype} n={n} ch={ch or 'default'}", flush=True)
    if ch:
        monkeypatch.setenv("QORA_HIP_TUNING", "1")   # the library reads tuning variables only then
        monkeypatch.setenv("QORA_HIP_PF_ATTN_CH", ch)
    if hd == 64:
        cfg = entry.smoke_config(pkg)
    else:
        cfg = pkg.ModelConfig(num_layers=2, vocab=1000, hidden=256, intermediate=704, num_heads=16,
                              num_kv_heads=4, head_dim=128, rope_half_dim=64, rope_theta=5e6, rope_positions=512)
    cfg.num_layers = 4
    cfg.rope_positions = 512
    w = pkg.synthetic_model(cfg, seed=4, fmt=1, rope_positions=512)
    prompt = pkg.synth_tokens(4, 2800 + n, n, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=512, kv_dtype=kv_dtype)
    om = orc.OracleModel(w, kv_capacity=512, T=4)
    tol = REL_TOL if kv_dtype == 0 else 5e-3
    logits, _ = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= tol
    for layer in (0, 3):
        k, v = be.kv_layer(layer)
        kr, vr = om.kv_layer(layer)
        assert rel_err(k, kr) <= tol and rel_err(v, vr) <= tol
    t = pkg.synth_tokens(4, 2900, 1, w.config.vocab)[0]
    logits, _ = be.forward_decode_raw(int(t))
    assert rel_err(logits, om.forward_decode(int(t))) <= tol


def test_batched_prefill_attention_many_keys(ctx, pkg, orc):
    """1100 tokens: the third 512-token chunk attends to 1100 keys, more than
    8 chunks of 128, so the chunk grows to 192 keys (6 chunks)."""
    print("case prefill key chunks 1100 tokens", flush=True)
    w = _model(pkg, 1, layers=2, seed=8, positions=1200)
    prompt = pkg.synth_tokens(8, 3000, 1100, w.config.vocab)
    be = pkg.HipBackend(ctx, w, kv_capacity=1200)
    om = orc.OracleModel(w, kv_capacity=1200, T=8)
    logits, _ = be.raw_prefill(prompt)
    assert rel_err(logits, om.prefill(prompt)) <= REL_TOL
    k, v = be.kv_layer(1)
    kr, vr = om.kv_layer(1)
    assert rel_err(k, kr) <= REL_TOL and rel_err(v, vr) <= REL_TOL
