"""The allocation-free GEMV entry (qora_hip_gemv_q4_noalloc) against the
entry it mirrors (qora_hip_gemv_q4): the same kernels on a static device
scratch array instead of the context's accumulator, so the outputs are
bit-identical. Two calls in a row, the second with a smaller output, then
a size beyond the array, which is refused."""
import numpy as np
import pytest

from helpers import device

pytestmark = pytest.mark.gpu


def _run(ctx, d, fn, packed, scales, x, k, n):
    y = d.empty(n * 4)
    rc = fn(ctx.h, d.put(packed), d.put(scales), d.put(x), y, k, n, None)
    ctx.check(rc, fn.__name__)
    return d.get(y, n, np.float32)


def test_noalloc_gemv_matches_gemv_q4(ctx, pkg):
    print("case gemv_q4_noalloc vs gemv_q4", flush=True)
    with device(ctx) as d:
        for (k, n) in ((2048, 11008), (300, 352)):          # the second call is smaller
            packed, scales = pkg.synth_q4(61, k + n, k, n)
            x = pkg.synth_f32(61, 7, k)
            want = _run(ctx, d, ctx.lib.qora_hip_gemv_q4, packed, scales, x, k, n)
            got = _run(ctx, d, ctx.lib.qora_hip_gemv_q4_noalloc, packed, scales, x, k, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (k, n)
            assert np.any(got != 0)


def test_noalloc_gemv_refuses_sizes_beyond_its_scratch(ctx, pkg):
    print("case gemv_q4_noalloc size limit", flush=True)
    k, n = 64, 65536 + 32
    packed, scales = pkg.synth_q4(62, 1, k, n)
    x = pkg.synth_f32(62, 2, k)
    with device(ctx) as d:
        y = d.empty(n * 4)
        rc = ctx.lib.qora_hip_gemv_q4_noalloc(ctx.h, d.put(packed), d.put(scales), d.put(x), y, k, n, None)
        assert rc == pkg.QORA_HIP_E_INVALID
        # the largest size it takes still runs
        n2 = 65536
        packed2, scales2 = pkg.synth_q4(62, 3, k, n2)
        want = _run(ctx, d, ctx.lib.qora_hip_gemv_q4, packed2, scales2, x, k, n2)
        got = _run(ctx, d, ctx.lib.qora_hip_gemv_q4_noalloc, packed2, scales2, x, k, n2)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_gemv_refused_call_launches_nothing(ctx, pkg):
    """Arguments are checked before the first launch: a refused call (n not a
    multiple of 32, a null input) returns QORA_HIP_E_INVALID and enqueues no
    write to the shared scratch, so a result computed around it is intact."""
    print("case gemv_q4_noalloc refused calls", flush=True)
    k, n = 2048, 2048
    packed, scales = pkg.synth_q4(63, 1, k, n)
    x = pkg.synth_f32(63, 2, k)
    with device(ctx) as d:
        want = _run(ctx, d, ctx.lib.qora_hip_gemv_q4, packed, scales, x, k, n)
        pk, sc, xd = d.put(packed), d.put(scales), d.put(x)
        y = d.empty(n * 4)
        ctx.check(ctx.lib.qora_hip_gemv_q4_noalloc(ctx.h, pk, sc, xd, y, k, n, None), "noalloc")
        # queued behind the valid call on the same stream, before its result is read
        assert ctx.lib.qora_hip_gemv_q4_noalloc(ctx.h, pk, sc, xd, d.empty(48 * 4), k, 48, None) == \
            pkg.QORA_HIP_E_INVALID
        assert ctx.lib.qora_hip_gemv_q4_noalloc(ctx.h, pk, sc, None, d.empty(64 * 4), k, 64, None) == \
            pkg.QORA_HIP_E_INVALID
        got = d.get(y, n, np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
