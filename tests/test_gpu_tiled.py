"""The decode step's GEMV on the tile layout, through qora_hip_gemv_prepare/run.

Q4 runs on the integer matrix cores (exact integer sums of x*s quantised to
30 bits against a block exponent): outputs are compared with the oracle at
REL_TOL (max error over max |reference|) and with the float64 truth at
TRUTH_TOL, bit-exactly in the exact-arithmetic regime (power-of-two scales,
small integer inputs), and exactly zero where the weights are all q = 8.
F16 runs on the VALU kernel, whose tile layout only reorders bytes: its
sums are compared bit-exactly with the reference-layout entry point."""
import numpy as np
import pytest

from helpers import REL_TOL, device, dequant_np, elem_err, exact_q4, rel_err

pytestmark = pytest.mark.gpu

FIX = 2.0 ** 36
# The MFMA path's only rounding is the 30-bit quantisation of x*s (2^-30 of
# the block bound per term): well below fp32 accumulation error.
TRUTH_TOL = 2e-6
SHAPES = [(2048, 11008), (11008, 2048), (2048, 2048), (2048, 512), (1, 32), (3, 96), (37, 224), (300, 352),
          (513, 64), (4097, 1056)]
PAIRED = [(2048, 11008), (2048, 1024), (37, 224), (513, 96), (1, 32)]


def _upload_q4(ctx, pkg, packed, scales, k, n):
    return ctx.upload(pkg.Weight(k=k, n=n, packed=packed, scales=scales))


def _run_prepared(ctx, d, gid, x, nacc):
    xd = d.put(x.astype(np.float32))
    acc = d.put(np.zeros(nacc, np.int64))
    ctx.gemv_run(gid, xd, acc)
    return d.get(acc, nacc, np.int64)


@pytest.mark.parametrize("k,n", SHAPES)
def test_prepared_q4_vs_oracle_and_truth(ctx, orc, pkg, k, n):
    print(f"case prepared q4 k={k} n={n}", flush=True)
    packed, scales = pkg.synth_q4(11, 5, k, n)
    x = pkg.synth_f32(11, 6, k)
    gid = ctx.gemv_prepare(_upload_q4(ctx, pkg, packed, scales, k, n))
    try:
        with device(ctx) as d:
            acc = _run_prepared(ctx, d, gid, x, n)
    finally:
        ctx.gemv_release(gid)
    y = acc / FIX
    wd = dequant_np(packed, scales, k, n)
    mag = np.abs(wd).T @ np.abs(x.astype(np.float64))     # each output's own scale
    for T in (1, 12):
        ref = orc.gemv_q4(x, packed, scales, k, n, T=T)
        assert rel_err(y, ref) <= REL_TOL
        assert elem_err(y, ref, mag) <= REL_TOL
    truth = wd.T @ x.astype(np.float64)
    assert rel_err(y, truth) <= TRUTH_TOL
    assert elem_err(y, truth, mag) <= TRUTH_TOL


@pytest.mark.parametrize("k,n", [(2048, 2048), (37, 224), (4097, 1056)])
def test_prepared_q4_exact_regime(ctx, pkg, k, n):
    r = np.random.default_rng(k + n)
    packed, scales = exact_q4(r, k, n)
    x = r.integers(-4, 5, size=k).astype(np.float32)
    truth = dequant_np(packed, scales, k, n).T @ x.astype(np.float64)
    gid = ctx.gemv_prepare(_upload_q4(ctx, pkg, packed, scales, k, n))
    try:
        with device(ctx) as d:
            acc = _run_prepared(ctx, d, gid, x, n)
    finally:
        ctx.gemv_release(gid)
    assert np.array_equal(acc / FIX, truth)


def test_prepared_q4_zero_cases(ctx, pkg):
    k, n = 256, 512
    packed, scales = pkg.synth_q4(3, 1, k, n)
    gid = ctx.gemv_prepare(_upload_q4(ctx, pkg, packed, scales, k, n))
    gid8 = ctx.gemv_prepare(_upload_q4(ctx, pkg, np.full_like(packed, 0x88), scales, k, n))
    try:
        with device(ctx) as d:
            assert not np.any(_run_prepared(ctx, d, gid, np.zeros(k, np.float32), n))
            assert not np.any(_run_prepared(ctx, d, gid8, pkg.synth_f32(3, 2, k) * 100, n))
    finally:
        ctx.gemv_release(gid)
        ctx.gemv_release(gid8)


@pytest.mark.parametrize("k,n", PAIRED)
def test_prepared_gate_up_vs_oracle_and_truth(ctx, orc, pkg, k, n):
    print(f"case prepared gate_up k={k} n={n}", flush=True)
    gp, gs = pkg.synth_q4(12, 1, k, n)
    up, us = pkg.synth_q4(12, 2, k, n)
    x = pkg.synth_f32(12, 3, k)
    gid = ctx.gemv_prepare(_upload_q4(ctx, pkg, gp, gs, k, n), _upload_q4(ctx, pkg, up, us, k, n), paired=True)
    try:
        with device(ctx) as d:
            acc = _run_prepared(ctx, d, gid, x, 2 * n)
    finally:
        ctx.gemv_release(gid)
    for half, (pk, sc) in enumerate(((gp, gs), (up, us))):
        y = acc[half * n:(half + 1) * n] / FIX
        assert rel_err(y, orc.gemv_q4(x, pk, sc, k, n, T=1)) <= REL_TOL
        assert rel_err(y, dequant_np(pk, sc, k, n).T @ x.astype(np.float64)) <= TRUTH_TOL


@pytest.mark.parametrize("k,n", [(2048, 2048), (300, 352)])
def test_prepared_q4_scale_extremes(ctx, pkg, k, n):
    """Block exponents over mixed magnitudes: inputs spanning 2^-20..2^6 and
    scales from binary16 denormals to 2^4, chosen so every output stays in
    the fixed-point accumulator range (|v| < 2^27)."""
    r = np.random.default_rng(k * 3 + n)
    packed, _ = pkg.synth_q4(16, 1, k, n)
    e = r.integers(-24, 4, size=k * n // 32)
    scales = (r.choice([-1.0, 1.0], size=e.size) * 2.0 ** e * r.uniform(1, 2, size=e.size)).astype(np.float16)
    scales = scales.view(np.uint16)
    x = (r.normal(size=k) * 2.0 ** r.integers(-20, 6, size=k)).astype(np.float32)
    gid = ctx.gemv_prepare(_upload_q4(ctx, pkg, packed, scales, k, n))
    try:
        with device(ctx) as d:
            acc = _run_prepared(ctx, d, gid, x, n)
    finally:
        ctx.gemv_release(gid)
    truth = dequant_np(packed, scales, k, n).T @ x.astype(np.float64)
    assert np.max(np.abs(truth)) < 2.0 ** 27
    # the block bound max|x| * max|s| can exceed the largest product of the
    # slice by several bits when magnitudes are mixed this widely
    err = rel_err(acc / FIX, truth)
    print(f"scale extremes k={k} n={n}: rel err vs float64 {err:.2e}", flush=True)
    assert err <= 2e-5


# F16 fp32 accumulation of k terms against the float64 truth (normwise)
F16_TRUTH_TOL = 1e-5


@pytest.mark.parametrize("k,n", [(2048, 2048), (300, 352), (2048, 512), (11008, 2048), (2048, 11008)])
def test_prepared_f16_vs_oracle(ctx, orc, pkg, k, n):
    print(f"case prepared f16 k={k} n={n}", flush=True)
    w = pkg.synth_f16(13, 1, k * n, 0.02)
    x = pkg.synth_f32(13, 2, k)
    wid = ctx.upload(pkg.Weight(k=k, n=n, data=w))
    gid = ctx.gemv_prepare(wid)
    try:
        with device(ctx) as d:
            acc = _run_prepared(ctx, d, gid, x, n)
            # the reference-layout entry (clear, accumulate, convert) must agree exactly
            y = d.empty(n * 4)
            wp, _ = ctx.weight_ptrs(wid)
            ctx.check(ctx.lib.qora_hip_gemv_f16(ctx.h, wp, d.put(x), y, k, n, None), "gemv_f16")
            y_ref_layout = d.get(y, n, np.float32)
    finally:
        ctx.gemv_release(gid)
    assert np.array_equal((acc / FIX).astype(np.float32), y_ref_layout)
    for avx in (False, True):
        assert rel_err(acc / FIX, orc.gemv_f16(x, w, k, n, avx512=avx)) <= REL_TOL
    wd = w.view(np.float16).astype(np.float64).reshape(k, n)
    truth = wd.T @ x.astype(np.float64)
    assert rel_err(acc / FIX, truth) <= F16_TRUTH_TOL
    assert elem_err(acc / FIX, truth, np.abs(wd).T @ np.abs(x.astype(np.float64))) <= F16_TRUTH_TOL


@pytest.mark.parametrize("k,n", [(2048, 11008), (37, 224)])
def test_prepared_f16_gate_up_vs_oracle_and_truth(ctx, orc, pkg, k, n):
    """The paired F16 GEMV of the decode step's gate|up launch (gate at
    acc[0:n], up at acc[n:2n]) at the model's 2048 -> 2 x 11008 shape."""
    print(f"case prepared f16 gate_up k={k} n={n}", flush=True)
    gw = pkg.synth_f16(17, 1, k * n, 0.02)
    uw = pkg.synth_f16(17, 2, k * n, 0.02)
    x = pkg.synth_f32(17, 3, k)
    gid = ctx.gemv_prepare(ctx.upload(pkg.Weight(k=k, n=n, data=gw)), ctx.upload(pkg.Weight(k=k, n=n, data=uw)),
                           paired=True)
    try:
        with device(ctx) as d:
            acc = _run_prepared(ctx, d, gid, x, 2 * n)
    finally:
        ctx.gemv_release(gid)
    for half, wh in enumerate((gw, uw)):
        y = acc[half * n:(half + 1) * n] / FIX
        for avx in (False, True):
            assert rel_err(y, orc.gemv_f16(x, wh, k, n, avx512=avx)) <= REL_TOL
        truth = wh.view(np.float16).astype(np.float64).reshape(k, n).T @ x.astype(np.float64)
        assert rel_err(y, truth) <= F16_TRUTH_TOL


def test_prepared_graph_replay(ctx, pkg):
    k, n = 2048, 2048
    packed, scales = pkg.synth_q4(14, 1, k, n)
    x = pkg.synth_f32(14, 2, k)
    gid = ctx.gemv_prepare(_upload_q4(ctx, pkg, packed, scales, k, n))
    try:
        with device(ctx) as d:
            once = _run_prepared(ctx, d, gid, x, n)
            xd = d.put(x)
            acc = d.put(np.zeros(n, np.int64))
            ctx.capture_begin()
            ctx.gemv_run(gid, xd, acc, ctx.stream)
            g = ctx.capture_end()
            try:
                for rep in range(1, 4):
                    ctx.graph_launch(g)
                    ctx.synchronize()
                    assert np.array_equal(d.get(acc, n, np.int64), once * rep)
            finally:
                ctx.graph_destroy(g)
    finally:
        ctx.gemv_release(gid)


def test_prepared_errors(ctx, pkg):
    packed, scales = pkg.synth_q4(15, 1, 64, 64)
    a = _upload_q4(ctx, pkg, packed, scales, 64, 64)
    packed2, scales2 = pkg.synth_q4(15, 2, 64, 96)
    b = _upload_q4(ctx, pkg, packed2, scales2, 64, 96)
    with pytest.raises(pkg.QoraHipError):
        ctx.gemv_prepare(a, b, paired=True)          # gate/up shapes differ
    with pytest.raises(pkg.QoraHipError):
        ctx.gemv_prepare(10 ** 6)                    # unknown weight
    gid = ctx.gemv_prepare(a)
    ctx.gemv_release(gid)
    with pytest.raises(pkg.QoraHipError):
        ctx.gemv_release(gid)                        # released twice
    with device(ctx) as d:
        with pytest.raises(pkg.QoraHipError):
            ctx.gemv_run(gid, d.put(np.zeros(64, np.float32)), d.put(np.zeros(64, np.int64)))
