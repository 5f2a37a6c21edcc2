"""Kernel-level parity on the GPU, through the C ABI, against the oracle.

Bars: bit-exact for dequant and for the exact-arithmetic GEMV regime;
max relative error REL_TOL = 1e-3 (normalised by max |reference|) for
floating-point outputs at fp32 accumulation."""
import ctypes

import numpy as np
import pytest

from helpers import REL_TOL, dequant_np, device, elem_err, exact_q4, random_q4, rel_err, rng

pytestmark = pytest.mark.gpu


def _gemv_q4(ctx, d, packed, scales, x, k, n):
    y = d.empty(n * 4)
    ctx.check(ctx.lib.qora_hip_gemv_q4(ctx.h, d.put(packed), d.put(scales), d.put(x.astype(np.float32)), y, k, n,
                                       None), "gemv_q4")
    return d.get(y, n, np.float32)


# real SmolLM3 projection shapes (k, n) and small ragged ones
Q4_SHAPES = [(2048, 11008), (11008, 2048), (2048, 2048), (2048, 512), (1, 32), (3, 96), (37, 224), (300, 352),
             (513, 64), (4097, 1056)]


@pytest.mark.parametrize("k,n", Q4_SHAPES)
def test_gemv_q4_exact_regime_bit_exact(ctx, orc, k, n):
    r = rng(k * 7 + n)
    packed, scales = exact_q4(r, k, n)
    x = r.integers(-4, 5, size=k).astype(np.float32)
    truth = dequant_np(packed, scales, k, n).T @ x.astype(np.float64)
    with device(ctx) as d:
        y = _gemv_q4(ctx, d, packed, scales, x, k, n)
    ref = orc.gemv_q4(x, packed, scales, k, n, T=4)
    assert np.array_equal(ref.astype(np.float64), truth)
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("k,n", Q4_SHAPES)
def test_gemv_q4_random_vs_oracle(ctx, orc, pkg, k, n):
    packed, scales = pkg.synth_q4(0, 7, k, n)
    x = pkg.synth_f32(0, 99, k)
    with device(ctx) as d:
        y = _gemv_q4(ctx, d, packed, scales, x, k, n)
    for T in (1, 12):
        ref = orc.gemv_q4(x, packed, scales, k, n, T=T)
        assert rel_err(y, ref) <= REL_TOL, (T, rel_err(y, ref))
    wd = dequant_np(packed, scales, k, n)
    truth = wd.T @ x.astype(np.float64)
    assert rel_err(y, truth) <= 1e-5
    assert elem_err(y, truth, np.abs(wd).T @ np.abs(x.astype(np.float64))) <= 1e-5


def test_gemv_q4_one_hot_is_dequant_row(ctx, orc):
    k, n = 300, 352
    r = rng(3)
    packed, scales = random_q4(r, k, n)
    deq = orc.dequant_q4(packed, scales, k, n)
    with device(ctx) as d:
        for i in (0, 1, 150, 299):
            x = np.zeros(k, dtype=np.float32)
            x[i] = 1.0
            y = _gemv_q4(ctx, d, packed, scales, x, k, n)
            assert np.array_equal(y, deq[i])


def test_gemv_q4_zero_cases(ctx):
    k, n = 128, 256
    r = rng(4)
    packed, scales = random_q4(r, k, n)
    with device(ctx) as d:
        y = _gemv_q4(ctx, d, packed, scales, np.zeros(k, np.float32), k, n)
        assert not np.any(y)
        y = _gemv_q4(ctx, d, np.full_like(packed, 0x88), scales, r.normal(size=k).astype(np.float32), k, n)
        assert not np.any(y)
        y = _gemv_q4(ctx, d, packed, np.zeros_like(scales), r.normal(size=k).astype(np.float32), k, n)
        assert not np.any(y)


def test_gemv_q4_linear_in_x(ctx):
    k, n = 2048, 2048
    r = rng(5)
    packed, scales = exact_q4(r, k, n)
    a = r.integers(-3, 4, size=k).astype(np.float32)
    b = r.integers(-3, 4, size=k).astype(np.float32)
    with device(ctx) as d:
        ya = _gemv_q4(ctx, d, packed, scales, a, k, n)
        yb = _gemv_q4(ctx, d, packed, scales, b, k, n)
        yab = _gemv_q4(ctx, d, packed, scales, a + b, k, n)
    assert np.array_equal(ya + yb, yab)


def test_gemv_q4_rejects_bad_shapes(ctx, pkg):
    with device(ctx) as d:
        p = d.empty(1024)
        for k, n in ((0, 32), (4, 0), (4, 33)):
            rc = ctx.lib.qora_hip_gemv_q4(ctx.h, p, p, p, p, k, n, None)
            assert rc == pkg.QORA_HIP_E_INVALID
        assert ctx.lib.qora_hip_gemv_q4(ctx.h, None, p, p, p, 4, 32, None) == pkg.QORA_HIP_E_INVALID


def test_dequant_q4_exhaustive_bit_exact(ctx, orc):
    # every byte value against special scales: +-0, subnormal, min normal, 1, max
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x2E66],
                        dtype=np.uint16)
    k, n = len(specials), 512
    packed = np.tile(np.arange(256, dtype=np.uint8), k)
    scales = np.repeat(specials, n // 32)
    truth = dequant_np(packed, scales, k, n).astype(np.float32)
    with device(ctx) as d:
        out = d.empty(k * n * 4)
        ctx.check(ctx.lib.qora_hip_dequant_q4(ctx.h, d.put(packed), d.put(scales), k, n, out, None), "dequant")
        got = d.get(out, (k, n), np.float32)
    ref = orc.dequant_q4(packed, scales, k, n)
    assert np.array_equal(ref.view(np.uint32), truth.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_q4_synthetic_bit_exact(ctx, orc, pkg):
    k, n = 2048, 11008
    packed, scales = pkg.synth_q4(0, 4, k, n)
    with device(ctx) as d:
        out = d.empty(k * n * 4)
        ctx.check(ctx.lib.qora_hip_dequant_q4(ctx.h, d.put(packed), d.put(scales), k, n, out, None), "dequant")
        got = d.get(out, (k, n), np.float32)
    assert np.array_equal(got, orc.dequant_q4(packed, scales, k, n))


ROWDOT_SHAPES = [(128256, 2048), (1000, 256), (77, 64), (5, 32), (3, 1024)]


@pytest.mark.parametrize("rows,cols", ROWDOT_SHAPES)
def test_rowdot_q4_vs_oracle_lm_head(ctx, orc, pkg, rows, cols):
    packed, scales = pkg.synth_q4(1, 1000, rows, cols)
    x = pkg.synth_f32(1, 98, cols)
    with device(ctx) as d:
        y = d.empty(rows * 4)
        ctx.check(ctx.lib.qora_hip_gemv_q4_rowdot(ctx.h, d.put(packed), d.put(scales), d.put(x), y, rows, cols, None),
                  "rowdot")
        got = d.get(y, rows, np.float32)
    ref = orc.lm_head_q4(x, packed, scales, rows, cols)
    assert rel_err(got, ref) <= REL_TOL
    wd = dequant_np(packed, scales, rows, cols)
    truth = wd @ x.astype(np.float64)
    assert rel_err(got, truth) <= 1e-5
    assert elem_err(got, truth, np.abs(wd) @ np.abs(x.astype(np.float64))) <= 1e-5


def test_rowdot_q4_exact_regime(ctx, orc):
    rows, cols = 4096, 2048
    r = rng(8)
    packed, scales = exact_q4(r, rows, cols)
    x = r.integers(-4, 5, size=cols).astype(np.float32)
    with device(ctx) as d:
        y = d.empty(rows * 4)
        ctx.check(ctx.lib.qora_hip_gemv_q4_rowdot(ctx.h, d.put(packed), d.put(scales), d.put(x), y, rows, cols, None),
                  "rowdot")
        got = d.get(y, rows, np.float32)
    assert np.array_equal(got, orc.lm_head_q4(x, packed, scales, rows, cols))


@pytest.mark.parametrize("k,n", [(2048, 11008), (64, 96), (100, 704), (33, 32)])
def test_gate_up_q4_vs_oracle(ctx, orc, pkg, k, n):
    gp, gs = pkg.synth_q4(2, 4, k, n)
    up, us = pkg.synth_q4(2, 5, k, n)
    x = pkg.synth_f32(2, 97, k) * 3.0
    with device(ctx) as d:
        out = d.empty(n * 4)
        ctx.check(ctx.lib.qora_hip_gate_up_q4(ctx.h, d.put(gp), d.put(gs), d.put(up), d.put(us), d.put(x), out, k, n,
                                              None), "gate_up")
        got = d.get(out, n, np.float32)
    for T in (1, 12):
        ref = orc.fused_gate_up_q4(x, gp, gs, up, us, k, n, T=T)
        assert rel_err(got, ref) <= REL_TOL, T


F16_SHAPES = [(2048, 11008), (11008, 2048), (2048, 512), (3, 96), (37, 224)]


@pytest.mark.parametrize("k,n", F16_SHAPES)
def test_gemv_f16_vs_oracle(ctx, orc, pkg, k, n):
    w = pkg.synth_f16(3, 6, k * n, 0.02)
    x = pkg.synth_f32(3, 96, k)
    with device(ctx) as d:
        y = d.empty(n * 4)
        ctx.check(ctx.lib.qora_hip_gemv_f16(ctx.h, d.put(w), d.put(x), y, k, n, None), "gemv_f16")
        got = d.get(y, n, np.float32)
    for avx in (1, 0):
        ref = orc.gemv_f16(x, w, k, n, T=12, avx512=avx)
        assert rel_err(got, ref) <= REL_TOL
    truth = w.view(np.float16).astype(np.float64).reshape(k, n).T @ x.astype(np.float64)
    assert rel_err(got, truth) <= 1e-5


def test_gate_up_f16_vs_oracle(ctx, orc, pkg):
    k, n = 2048, 11008
    gw = pkg.synth_f16(3, 7, k * n, 0.02)
    uw = pkg.synth_f16(3, 8, k * n, 0.02)
    x = pkg.synth_f32(3, 95, k)
    with device(ctx) as d:
        out = d.empty(n * 4)
        ctx.check(ctx.lib.qora_hip_gate_up_f16(ctx.h, d.put(gw), d.put(uw), d.put(x), out, k, n, None), "gate_up_f16")
        got = d.get(out, n, np.float32)
    assert rel_err(got, orc.fused_gate_up_f16(x, gw, uw, k, n, T=12)) <= REL_TOL
    g = gw.view(np.float16).astype(np.float64).reshape(k, n).T @ x.astype(np.float64)
    u = uw.view(np.float16).astype(np.float64).reshape(k, n).T @ x.astype(np.float64)
    assert rel_err(got, g / (1 + np.exp(-g)) * u) <= 1e-5


@pytest.mark.parametrize("rows,cols", [(128256, 2048), (32000, 2048), (1000, 256)])
def test_rowdot_f16_vs_oracle_lm_head(ctx, orc, pkg, rows, cols):
    """The F16 tied lm_head (row-dot, gemv.rs:805-822), up to the model's
    full 128256 x 2048 vocabulary."""
    print(f"case rowdot f16 rows={rows} cols={cols}", flush=True)
    w = pkg.synth_f16(4, 1000, rows * cols, 0.02)
    x = pkg.synth_f32(4, 94, cols)
    with device(ctx) as d:
        y = d.empty(rows * 4)
        ctx.check(ctx.lib.qora_hip_gemv_f16_rowdot(ctx.h, d.put(w), d.put(x), y, rows, cols, None), "rowdot_f16")
        got = d.get(y, rows, np.float32)
    assert rel_err(got, orc.lm_head_f16(x, w, rows, cols)) <= REL_TOL
    wm = w.view(np.float16).reshape(rows, cols)
    x64 = x.astype(np.float64)
    truth = np.concatenate([wm[r:r + 16384].astype(np.float64) @ x64 for r in range(0, rows, 16384)])
    assert rel_err(got, truth) <= 1e-5


@pytest.mark.parametrize("n", [2048, 11008, 1, 33])
def test_rmsnorm_vs_oracle(ctx, orc, pkg, n):
    x = pkg.synth_f32(5, 93, n) * 2.5
    gamma = (1.0 + 0.1 * pkg.synth_f32(5, 92, n)).astype(np.float16).view(np.uint16)
    with device(ctx) as d:
        out = d.empty(n * 4)
        ctx.check(ctx.lib.qora_hip_rmsnorm(ctx.h, d.put(x), d.put(gamma), n, out, None), "rmsnorm")
        got = d.get(out, n, np.float32)
    assert rel_err(got, orc.rms_norm(x, gamma)) <= 1e-5


def test_rmsnorm_constant_closed_form(ctx):
    n, c = 2048, 0.75
    x = np.full(n, c, dtype=np.float32)
    gamma = np.full(n, 0x3C00, dtype=np.uint16)
    with device(ctx) as d:
        out = d.empty(n * 4)
        ctx.check(ctx.lib.qora_hip_rmsnorm(ctx.h, d.put(x), d.put(gamma), n, out, None), "rmsnorm")
        got = d.get(out, n, np.float32)
    assert np.allclose(got, c / np.sqrt(c * c + 1e-6), rtol=1e-6, atol=0)


@pytest.mark.parametrize("pos", [0, 5, 1000, 2047])
def test_rope_vs_oracle(ctx, orc, pkg, pos):
    heads, hd, half = 16, 128, 64
    cos_t, sin_t = pkg.rope_tables(2048, half, 5e6)
    data = pkg.synth_f32(6, 91, heads * hd)
    with device(ctx) as d:
        p = d.put(data)
        ctx.check(ctx.lib.qora_hip_rope(ctx.h, p, heads, hd, d.put(cos_t), d.put(sin_t), half, pos, None), "rope")
        got = d.get(p, heads * hd, np.float32)
    ref = orc.apply_rope(data, heads, hd, cos_t, sin_t, half, pos)
    assert rel_err(got, ref) <= 1e-6
    if pos == 0:
        assert np.array_equal(got, data)


@pytest.mark.parametrize("L", [1, 2, 31, 32, 33, 100, 2048, 2049, 5000, 32768])
@pytest.mark.parametrize("kv_f16", [0, 1])
def test_attention_vs_oracle(ctx, orc, pkg, L, kv_f16):
    H, KVH, hd = 16, 4, 128
    q = pkg.synth_f32(7, 90, H * hd)
    kc = pkg.synth_f32(7, 89, L * KVH * hd)
    vc = pkg.synth_f32(7, 88, L * KVH * hd)
    if kv_f16:
        kd, vd = kc.astype(np.float16), vc.astype(np.float16)
        kref, vref = kd.astype(np.float32), vd.astype(np.float32)
        kdev, vdev = kd.view(np.uint16), vd.view(np.uint16)
    else:
        kref, vref, kdev, vdev = kc, vc, kc, vc
    with device(ctx) as d:
        out = d.empty(H * hd * 4)
        ctx.check(ctx.lib.qora_hip_attn_decode(ctx.h, d.put(q), d.put(kdev), d.put(vdev), kv_f16, L, H, KVH, hd, out,
                                               None), "attn")
        got = d.get(out, H * hd, np.float32)
    ref = orc.attention_decode(q, kref, vref, L, H, KVH, hd)
    assert rel_err(got, ref) <= REL_TOL
    if L == 1:
        # one position: softmax weight 1, output = V of the head's KV head
        v = vref.reshape(KVH, hd)
        assert np.allclose(got.reshape(H, hd), np.repeat(v, H // KVH, axis=0), rtol=1e-6, atol=1e-7)


def test_attention_identical_keys_mean_of_v_and_gqa_mapping(ctx, pkg):
    H, KVH, hd, L = 16, 4, 128, 50
    q = pkg.synth_f32(8, 87, H * hd)
    krow = pkg.synth_f32(8, 86, KVH * hd)
    kc = np.tile(krow, L)
    # head-distinct V: V[s][kvh][d] = 100*kvh + s
    vc = (100.0 * np.arange(KVH)[None, :, None] + np.arange(L)[:, None, None] + np.zeros((1, 1, hd))).astype(
        np.float32).reshape(-1)
    with device(ctx) as d:
        out = d.empty(H * hd * 4)
        ctx.check(ctx.lib.qora_hip_attn_decode(ctx.h, d.put(q), d.put(kc), d.put(vc), 0, L, H, KVH, hd, out, None),
                  "attn")
        got = d.get(out, (H, hd), np.float32)
    expect = 100.0 * (np.arange(H) // (H // KVH)) + (L - 1) / 2.0
    assert np.allclose(got, expect[:, None], rtol=1e-5)


def _argmax(ctx, d, logits):
    out = d.empty(4)
    ctx.check(ctx.lib.qora_hip_argmax(ctx.h, d.put(logits.astype(np.float32)), logits.size, out, None), "argmax")
    return int(d.get(out, 1, np.int32)[0])


def test_argmax_first_max_rule(ctx, orc):
    with device(ctx) as d:
        x = np.zeros(128256, dtype=np.float32)
        x[[7, 100, 128000]] = 5.0
        assert _argmax(ctx, d, x) == 7 == orc.argmax(x)
        x = np.full(1000, -np.inf, dtype=np.float32)
        assert _argmax(ctx, d, x) == 0 == orc.argmax(x)
        x[0] = np.nan
        x[500] = -1e30
        assert _argmax(ctx, d, x) == 500 == orc.argmax(x)
        x = np.full(1000, np.nan, dtype=np.float32)
        assert _argmax(ctx, d, x) == 0 == orc.argmax(x)
        x = np.random.default_rng(1).normal(size=128256).astype(np.float32)
        assert _argmax(ctx, d, x) == orc.argmax(x) == int(np.argmax(x))


def test_graph_capture_replays_match_eager(ctx, pkg, orc):
    """Captured kernel-level calls replayed several times, with eager work and
    synchronisations between the replays; every replay equals the eager result."""
    k, n = 2048, 11008
    gp, gs = pkg.synth_q4(9, 4, k, n)
    up, us = pkg.synth_q4(9, 5, k, n)
    x = pkg.synth_f32(9, 85, k)
    with device(ctx) as d:
        pg, sg, pu, su, px = d.put(gp), d.put(gs), d.put(up), d.put(us), d.put(x)
        out = d.empty(n * 4)
        ctx.check(ctx.lib.qora_hip_gate_up_q4(ctx.h, pg, sg, pu, su, px, out, k, n, None), "eager")
        eager = d.get(out, n, np.float32)
        ctx.capture_begin()
        ctx.check(ctx.lib.qora_hip_gate_up_q4(ctx.h, pg, sg, pu, su, px, out, k, n, None), "captured")
        g = ctx.capture_end()
        try:
            for i in range(4):
                ctx.h2d(out, np.zeros(n, np.float32))
                ctx.graph_launch(g, 1)
                ctx.synchronize()
                assert np.array_equal(d.get(out, n, np.float32), eager), i
                y2 = d.empty(n * 4)
                ctx.check(ctx.lib.qora_hip_gemv_q4(ctx.h, pg, sg, px, y2, k, n, None), "eager between")
        finally:
            ctx.graph_destroy(g)
