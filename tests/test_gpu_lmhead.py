"""The decode step's tied lm_head on the matrix cores, through
qora_hip_lm_head_prepare / qora_hip_lm_head_run.

Logits are compared with the oracle's lm_head_q4 (gemv.rs:825-864) at REL_TOL
and with the float64 truth at TRUTH_TOL, bit-exactly in the exact-arithmetic
regime; the greedy index with the first-max rule (generate.rs:346-352)."""
import ctypes

import numpy as np
import pytest

from helpers import REL_TOL, device, dequant_np, exact_q4, rel_err, rng

pytestmark = pytest.mark.gpu

# Exact integer group sums, then fp32: each 64-column block's value and the
# running sum round once per step, like fp32 accumulation.
TRUTH_TOL = 1e-5
SHAPES = [(128256, 2048), (1000, 256), (37, 128), (4097, 512), (16, 1024), (17, 2048)]


def _run(ctx, d, lid, x, rows, want_argmax=True):
    xd = d.put(x.astype(np.float32))
    y = d.empty(rows * 4)
    am = d.put(np.full(1, -5, np.int32)) if want_argmax else 0
    ctx.lm_head_run(lid, xd, y, am)
    logits = d.get(y, rows, np.float32)
    tok = int(d.get(am, 1, np.int32)[0]) if want_argmax else None
    return logits, tok


def first_max(v):
    ok = v > -np.inf
    if not np.any(ok):
        return 0
    best = np.max(v[ok])
    return int(np.flatnonzero(v == best)[0])


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_lm_head_vs_oracle_and_truth(ctx, orc, pkg, rows, cols):
    print(f"case lm_head rows={rows} cols={cols}", flush=True)
    packed, scales = pkg.synth_q4(21, 1, rows, cols)
    x = pkg.synth_f32(21, 2, cols)
    wid = ctx.upload(pkg.Weight(k=rows, n=cols, packed=packed, scales=scales))
    lid = ctx.lm_head_prepare(wid)
    try:
        with device(ctx) as d:
            logits, tok = _run(ctx, d, lid, x, rows)
    finally:
        ctx.gemv_release(lid)
    ref = orc.lm_head_q4(x, packed, scales, rows, cols)
    assert rel_err(logits, ref) <= REL_TOL
    truth = dequant_np(packed, scales, rows, cols) @ x.astype(np.float64)
    err = rel_err(logits, truth)
    print(f"lm_head {rows}x{cols}: rel err vs float64 {err:.2e}", flush=True)
    assert err <= TRUTH_TOL
    assert tok == first_max(logits)
    top = np.sort(truth)[-2:]
    if top[1] - top[0] > 1e-4 * abs(top[1]):
        assert tok == orc.argmax(ref) == int(np.argmax(truth))


@pytest.mark.parametrize("rows,cols", [(4096, 2048), (300, 256)])
def test_lm_head_exact_regime(ctx, pkg, rows, cols):
    r = rng(rows + cols)
    packed, scales = exact_q4(r, rows, cols)
    x = r.integers(-4, 5, size=cols).astype(np.float32)
    truth = dequant_np(packed, scales, rows, cols) @ x.astype(np.float64)
    wid = ctx.upload(pkg.Weight(k=rows, n=cols, packed=packed, scales=scales))
    lid = ctx.lm_head_prepare(wid)
    try:
        with device(ctx) as d:
            logits, tok = _run(ctx, d, lid, x, rows)
    finally:
        ctx.gemv_release(lid)
    assert np.array_equal(logits, truth.astype(np.float32))
    assert tok == first_max(logits)


def test_lm_head_zero_input_and_ties(ctx, pkg):
    rows, cols = 100, 256
    packed, scales = pkg.synth_q4(22, 1, rows, cols)
    wid = ctx.upload(pkg.Weight(k=rows, n=cols, packed=packed, scales=scales))
    lid = ctx.lm_head_prepare(wid)
    try:
        with device(ctx) as d:
            logits, tok = _run(ctx, d, lid, np.zeros(cols, np.float32), rows)
            assert not np.any(logits) and tok == 0          # all tie at 0: lowest index
            # rows 40 and 70 identical and largest: the lower one wins
            p2 = packed.reshape(rows, cols // 2).copy()
            s2 = scales.reshape(rows, cols // 32).copy()
            p2[:] = 0x88
            p2[40] = p2[70] = 0xFF
            s2[40] = s2[70] = np.float16(0.5).view(np.uint16)
            wid2 = ctx.upload(pkg.Weight(k=rows, n=cols, packed=p2.reshape(-1), scales=s2.reshape(-1)))
            lid2 = ctx.lm_head_prepare(wid2)
            try:
                logits2, tok2 = _run(ctx, d, lid2, np.ones(cols, np.float32), rows)
            finally:
                ctx.gemv_release(lid2)
    finally:
        ctx.gemv_release(lid)
    assert logits2[40] == logits2[70] == 0.5 * 7 * cols
    assert tok2 == 40


def test_lm_head_graph_replay(ctx, pkg):
    rows, cols = 5000, 2048
    packed, scales = pkg.synth_q4(23, 1, rows, cols)
    x = pkg.synth_f32(23, 2, cols)
    wid = ctx.upload(pkg.Weight(k=rows, n=cols, packed=packed, scales=scales))
    lid = ctx.lm_head_prepare(wid)
    try:
        with device(ctx) as d:
            once, tok = _run(ctx, d, lid, x, rows)
            xd = d.put(x)
            y = d.empty(rows * 4)
            am = d.put(np.zeros(1, np.int32))
            ctx.capture_begin()
            ctx.lm_head_run(lid, xd, y, am, ctx.stream)
            g = ctx.capture_end()
            try:
                for _ in range(3):
                    ctx.check(ctx.lib.qora_hip_memcpy_h2d(ctx.h, y, np.zeros(rows, np.float32).ctypes.data,
                                                          rows * 4), "clear")
                    ctx.graph_launch(g)
                    ctx.synchronize()
                    assert np.array_equal(d.get(y, rows, np.float32), once)
                    assert int(d.get(am, 1, np.int32)[0]) == tok
            finally:
                ctx.graph_destroy(g)
    finally:
        ctx.gemv_release(lid)


def test_lm_head_errors(ctx, pkg):
    packed, scales = pkg.synth_q4(24, 1, 64, 96)
    bad_cols = ctx.upload(pkg.Weight(k=64, n=96, packed=packed, scales=scales))
    f16 = ctx.upload(pkg.Weight(k=64, n=128, data=pkg.synth_f16(24, 2, 64 * 128, 0.02)))
    p2, s2 = pkg.synth_q4(24, 3, 64, 128)
    good = ctx.upload(pkg.Weight(k=64, n=128, packed=p2, scales=s2))
    for wid in (bad_cols, f16, 10 ** 6):
        with pytest.raises(pkg.QoraHipError):
            ctx.lm_head_prepare(wid)
    lid = ctx.lm_head_prepare(good)
    gid = ctx.gemv_prepare(good)
    try:
        with device(ctx) as d:
            x = d.put(np.zeros(128, np.float32))
            with pytest.raises(pkg.QoraHipError):
                ctx.gemv_run(lid, x, d.put(np.zeros(128, np.int64)))     # lm_head id on gemv_run
            with pytest.raises(pkg.QoraHipError):
                ctx.lm_head_run(gid, x, d.empty(64 * 4))                 # gemv id on lm_head_run
            with pytest.raises(pkg.QoraHipError):
                ctx.lm_head_run(lid, 0, d.empty(64 * 4))                 # null input
    finally:
        ctx.gemv_release(lid)
        ctx.gemv_release(gid)
    with pytest.raises(pkg.QoraHipError):
        ctx.gemv_release(lid)
