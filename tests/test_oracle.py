"""Pins of the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

The reference is Rust and cannot be built or imported here (no rustc/cargo),
and it ships no golden vectors, so each oracle function is pinned by
something independent of its own code:
  * numpy float32 restatements of the reference's operation order (numpy
    float32 rounds every operation, as the reference's scalar code does), so
    a reordered sum, a dropped term or a fused multiply-add fails bit-exactly;
  * float64 brute force and closed forms (one-hot rows, all-equal inputs,
    L = 1 attention, identical keys, exact-arithmetic regimes);
  * exhaustive enumeration where the domain is small (binary16, nibbles).
Functions whose bits depend on the platform's expf (SiLU, softmax) are
compared with tolerances: their bit-level parity is unpinned (the reference
calls Rust's f32::exp, i.e. the platform libm)."""
import numpy as np
import pytest

from helpers import dequant_np, exact_q4, random_q4, rel_err, rng
from model_f64 import F64Model

F32 = np.float32


# ---------------------------------------------------------------------------
# binary16 and nibbles
# ---------------------------------------------------------------------------

def test_h2f_exhaustive(orc):
    """half::f16::to_f32 (gemv.rs:450 etc.): exact IEEE binary16 widening, all 65536 codes."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([orc.h2f(int(c)) for c in codes], dtype=np.float32)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_q_minus_8_is_sign_extended_nibble():
    """q - 8 == sext4(q ^ 8) for every nibble (gpu_loader.rs:64-72), so the
    high-nibble byte trick 16*(q - 8) = ((q << 4) ^ 0x80) as int8 holds too."""
    for q in range(16):
        t = q ^ 8
        sext = t - 16 if t >= 8 else t
        assert sext == q - 8
        assert np.int8(np.uint8(((q << 4) & 0xF0) ^ 0x80)) == 16 * (q - 8)


def test_dequant_every_byte_and_scale_class(orc):
    """embed_lookup_q4 (gemv.rs:710-736): f32(scale) * (q - 8), exact, for all
    256 byte values against subnormal, signed zero, max and ordinary scales."""
    scale_codes = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x2E66,
                            0x1234, 0x5555], dtype=np.uint16)
    n = 32 * len(scale_codes)
    k = 16                                          # 16 rows x 16 bytes per group = all 256 bytes
    packed = np.zeros((k, n // 2), np.uint8)
    for r in range(k):
        for g in range(len(scale_codes)):
            packed[r, g * 16:(g + 1) * 16] = np.arange(16, dtype=np.uint8) + 16 * r
    scales = np.tile(scale_codes, k)
    got = orc.dequant_q4(packed.reshape(-1), scales, k, n)
    want = dequant_np(packed.reshape(-1), scales, k, n)
    assert np.array_equal(got, want.astype(np.float32))
    assert np.array_equal(got.astype(np.float64), want)          # exact in fp32


# ---------------------------------------------------------------------------
# Q4 GEMV
# ---------------------------------------------------------------------------

def q4_rows_f32(x, packed, scales, k, n, k0, k1):
    """gemv_q4_inner (gemv.rs:596-641) in numpy float32: per row, s = f32(scale)
    * x[row]; each element adds fl(s * (q - 8)); rows in order."""
    p = packed.reshape(k, n // 2)
    q = np.empty((k, n), np.int64)
    q[:, 0::2] = p & 15
    q[:, 1::2] = p >> 4
    qm8 = (q - 8).astype(F32)
    sc = scales.view(np.float16).astype(F32).reshape(k, n // 32)
    y = np.zeros(n, F32)
    for r in range(k0, k1):
        if x[r] == 0:
            continue
        s = np.repeat(sc[r] * F32(x[r]), 32)
        y = y + s * qm8[r]
    return y


def q4_gemv_f32(x, packed, scales, k, n, T):
    """gemv_q4 (gemv.rs:646-675): one pass when k*n < 4e6, else T chunks of
    ceil(k/T) rows summed onto zeros in thread order."""
    if k * n < 4_000_000 or T <= 1:
        return q4_rows_f32(x, packed, scales, k, n, 0, k)
    chunk = -(-k // T)
    out = np.zeros(n, F32)
    for t in range(T):
        ks, ke = t * chunk, min(k, (t + 1) * chunk)
        if ks >= k:
            continue
        out = out + q4_rows_f32(x, packed, scales, k, n, ks, ke)
    return out


@pytest.mark.parametrize("k,n", [(37, 96), (64, 64), (300, 352)])
def test_gemv_q4_single_pass_order_bit_exact(orc, pkg, k, n):
    packed, scales = pkg.synth_q4(5, 1, k, n)
    x = pkg.synth_f32(5, 2, k)
    x[3] = 0.0                                      # a skipped row
    want = q4_gemv_f32(x, packed, scales, k, n, 1)
    assert np.array_equal(orc.gemv_q4(x, packed, scales, k, n, T=1), want)


@pytest.mark.parametrize("T", [1, 3, 12])
def test_gemv_q4_k_split_order_bit_exact(orc, pkg, T):
    """The threaded form (k*n >= 4e6): partial sums per ceil(k/T)-row chunk."""
    k, n = 2048, 2048
    packed, scales = pkg.synth_q4(6, 1, k, n)
    x = pkg.synth_f32(6, 2, k)
    want = q4_gemv_f32(x, packed, scales, k, n, T)
    assert np.array_equal(orc.gemv_q4(x, packed, scales, k, n, T=T), want)


@pytest.mark.parametrize("k,n", [(64, 96), (2048, 2048), (513, 160)])
def test_gemv_q4_exact_regime(orc, k, n):
    """Power-of-two scales and small integer x: every partial sum is an exact
    integer times 2^-e, so any order gives the float64 truth exactly."""
    r = rng(k + n)
    packed, scales = exact_q4(r, k, n)
    x = r.integers(-4, 5, size=k).astype(F32)
    truth = dequant_np(packed, scales, k, n).T @ x.astype(np.float64)
    for T in (1, 7):
        assert np.array_equal(orc.gemv_q4(x, packed, scales, k, n, T=T).astype(np.float64), truth)


def test_gemv_q4_closed_forms(orc):
    k, n = 96, 128
    r = rng(9)
    packed, scales = random_q4(r, k, n)
    deq = orc.dequant_q4(packed, scales, k, n).reshape(k, n)
    for i in (0, 17, 95):                           # one-hot x -> that dequant row
        x = np.zeros(k, F32)
        x[i] = 1.0
        assert np.array_equal(orc.gemv_q4(x, packed, scales, k, n), deq[i])
    x = r.normal(size=k).astype(F32)
    assert not np.any(orc.gemv_q4(x, np.full_like(packed, 0x88), scales, k, n))      # q == 8
    assert not np.any(orc.gemv_q4(x, packed, np.zeros_like(scales), k, n))          # s == 0
    truth = dequant_np(packed, scales, k, n).T @ x.astype(np.float64)
    assert rel_err(orc.gemv_q4(x, packed, scales, k, n), truth) <= 1e-6


def test_gemv_q4_linear_in_x_exact_regime(orc):
    k, n = 128, 64
    r = rng(11)
    packed, scales = exact_q4(r, k, n)
    a = r.integers(-3, 4, size=k).astype(F32)
    b = r.integers(-3, 4, size=k).astype(F32)
    ya, yb = orc.gemv_q4(a, packed, scales, k, n), orc.gemv_q4(b, packed, scales, k, n)
    assert np.array_equal(orc.gemv_q4(a + b, packed, scales, k, n), ya + yb)
    assert np.array_equal(orc.gemv_q4(2 * a, packed, scales, k, n), 2 * ya)


def test_gemv_q4_row_range_matches_full(orc, pkg):
    k, n = 200, 96
    packed, scales = pkg.synth_q4(12, 1, k, n)
    x = pkg.synth_f32(12, 2, k)
    assert np.array_equal(orc.gemv_q4_rows(x, packed, scales, n, 50, 130),
                          q4_rows_f32(x, packed, scales, k, n, 50, 130))


# ---------------------------------------------------------------------------
# fused gate/up + SiLU, F16 GEMV, lm_head
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("T", [1, 5])
def test_fused_gate_up_vs_restatement(orc, pkg, T):
    """fused_gate_up_q4 (gemv.rs:412-502): always T chunk partials, then
    silu(g) * u. The partials are bit-exact through the restatement; SiLU's
    expf is the platform's, so the final step has a tolerance."""
    k, n = 160, 96
    gp, gs = pkg.synth_q4(13, 1, k, n)
    up, us = pkg.synth_q4(13, 2, k, n)
    x = pkg.synth_f32(13, 3, k)
    chunk = -(-k // T)
    g = np.zeros(n, F32)
    u = np.zeros(n, F32)
    for t in range(T):
        ks, ke = t * chunk, min(k, (t + 1) * chunk)
        if ks < ke:
            g = g + q4_rows_f32(x, gp, gs, k, n, ks, ke)
            u = u + q4_rows_f32(x, up, us, k, n, ks, ke)
    gd = g.astype(np.float64)
    want = gd / (1.0 + np.exp(-gd)) * u.astype(np.float64)
    got = orc.fused_gate_up_q4(x, gp, gs, up, us, k, n, T=T)
    assert rel_err(got, want) <= 1e-6


def test_gemv_f16_scalar_order_and_fma_form(orc, pkg):
    """gemv_f16 (gemv.rs:558-566): scalar path is y += fl(x * w), row by row
    (bit-exact restatement); the AVX-512 path (simd.rs:166) fuses the
    multiply-add, so it differs from the scalar one only in the last bits."""
    k, n = 96, 160
    w = pkg.synth_f16(14, 1, k * n, 0.02)
    x = pkg.synth_f32(14, 2, k)
    wf = w.view(np.float16).astype(F32).reshape(k, n)
    y = np.zeros(n, F32)
    for r in range(k):
        y = y + F32(x[r]) * wf[r]
    assert np.array_equal(orc.gemv_f16(x, w, k, n, avx512=False), y)
    truth = wf.astype(np.float64).T @ x.astype(np.float64)
    fma = orc.gemv_f16(x, w, k, n, avx512=True)
    assert rel_err(fma, truth) <= 1e-6
    assert not np.array_equal(fma, y) or k * n < 64    # the fused form is a different rounding


def test_lm_head_q4_row_dot_order(orc, pkg):
    """lm_head_parallel_q4 (gemv.rs:825-864): per row, lut[q] = scale*(q-8)
    (lut[8] = 0), dot += x[32g+2j] * lut[lo], then x[32g+2j+1] * lut[hi]."""
    vocab, hidden = 40, 64
    packed, scales = pkg.synth_q4(15, 1, vocab, hidden)
    scales[5] = 0                                   # a skipped group
    x = pkg.synth_f32(15, 2, hidden)
    G = hidden // 32
    want = np.zeros(vocab, F32)
    for v in range(vocab):
        dot = F32(0)
        for g in range(G):
            sc = np.uint16(scales[v * G + g]).view(np.float16).astype(F32)
            if sc == 0:
                continue
            lut = [F32(0) if q == 8 else F32(sc * F32(q - 8)) for q in range(16)]
            for j in range(16):
                b = int(packed[(v * G + g) * 16 + j])
                dot = F32(dot + F32(x[32 * g + 2 * j] * lut[b & 15]))
                dot = F32(dot + F32(x[32 * g + 2 * j + 1] * lut[b >> 4]))
        want[v] = dot
    assert np.array_equal(orc.lm_head_q4(x, packed, scales, vocab, hidden), want)


def fma_f32(a, b, c):
    """Correctly rounded float32 a*b + c (an FMA), elementwise, from float64:
    the product of two float32 values is exact in float64; TwoSum gives the
    exact error e of s = fl64(p + c); rounding s to float32 is then correct
    except when s lies exactly on a float32 midpoint and e != 0, where the
    sign of e decides: the exact sum s + e lies on the side e points to."""
    a64 = np.asarray(a, np.float64)
    b64 = np.asarray(b, np.float64)
    c64 = np.asarray(c, np.float64)
    p = a64 * b64
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(F32)
    d = s - r.astype(np.float64)
    nb = np.nextafter(r, np.where(d > 0, F32(np.inf), F32(-np.inf)).astype(F32))
    mid = (d != 0) & ((r.astype(np.float64) + nb.astype(np.float64)) * 0.5 == s)
    return np.where(mid & (e != 0) & (np.sign(e) == np.sign(d)), nb, r).astype(F32)


def test_fma_restatement_matches_libm_fmaf():
    """The FMA restatement against glibc's fmaf (correctly rounded), on random
    operands and on sums built to land exactly on float32 midpoints."""
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.fmaf.restype = ctypes.c_float
    libm.fmaf.argtypes = [ctypes.c_float] * 3
    r = rng(40)
    a = r.normal(size=4000).astype(F32)
    b = (r.normal(size=4000) * 0.02).astype(np.float16).astype(F32)
    c = (r.normal(size=4000) * 10.0 ** r.integers(-3, 4, size=4000)).astype(F32)
    # double-rounding cases: c has an odd last bit and a*b = h (1 - 2^-46),
    # h half an ulp of c, so fl64(a*b + c) is the float32 midpoint above c
    # (a tie that rounds to even, away from c) while the exact sum lies just
    # below it (correct result: c)
    cm = np.array([1 + 2.0 ** -23, 1 + 3 * 2.0 ** -23, 2 + 2.0 ** -22, 1000.0 + 2.0 ** -14], F32)
    am = np.full(cm.size, 1 + 2.0 ** -23, F32)
    bm = (np.spacing(cm) / 2 * (1 - 2.0 ** -23)).astype(F32)
    assert not np.array_equal((am.astype(np.float64) * bm + cm).astype(F32), cm)   # naive rounding is off
    for x, y, z in ((a, b, c), (am, bm, cm), (-am, bm, -cm)):
        want = np.array([libm.fmaf(float(p), float(q), float(t)) for p, q, t in zip(x, y, z)], F32)
        assert np.array_equal(fma_f32(x, y, z).view(np.uint32), want.view(np.uint32))


def f16_rows_fma(x, wf, n):
    """simd::gemv_f16_avx512 (simd.rs:151-176): rows with x == 0 skipped,
    out = fma(x, w, out) over the 16-aligned columns, out += x * w on the tail."""
    out = np.zeros(n, F32)
    n16 = n // 16 * 16
    for i in range(len(x)):
        if x[i] == 0:
            continue
        out[:n16] = fma_f32(F32(x[i]), wf[i, :n16], out[:n16])
        out[n16:] = out[n16:] + F32(x[i]) * wf[i, n16:]
    return out


def f16_gemv_avx(x, w, k, n, T):
    """gemv_f16's AVX-512 arm (gemv.rs:539-556): one pass when k*n < 4e6,
    else T partials of ceil(k/T) rows added onto zeros in thread order."""
    wf = w.view(np.float16).astype(F32).reshape(k, n)
    if k * n < 4_000_000:
        return f16_rows_fma(x, wf, n)
    chunk = -(-k // T)
    out = np.zeros(n, F32)
    for t in range(T):
        ks, ke = t * chunk, min(k, (t + 1) * chunk)
        if ks < ke:
            out = out + f16_rows_fma(x[ks:ke], wf[ks:ke], n)
    return out


@pytest.mark.parametrize("k,n,T", [(96, 160, 1), (40, 72, 1), (2048, 2048, 3), (2048, 2048, 12)])
def test_gemv_f16_avx_order_bit_exact(orc, pkg, k, n, T):
    """The AVX-512 F16 GEMV, single pass and k-split (k*n >= 4e6), bit-exact
    against the FMA restatement; n = 72 has a scalar tail."""
    w = pkg.synth_f16(41, k + n, k * n, 0.02)
    x = pkg.synth_f32(41, 2, k)
    x[5] = 0.0                                       # a skipped row
    want = f16_gemv_avx(x, w, k, n, T)
    assert np.array_equal(orc.gemv_f16(x, w, k, n, T=T, avx512=True).view(np.uint32), want.view(np.uint32))


def test_gate_up_f16_fallback(orc, pkg):
    """fused_gate_up_gemv with F16 weights (gemv.rs:395-407): two gemv_f16
    calls, then silu(g) * u (expf: tolerance)."""
    k, n = 64, 96
    gw = pkg.synth_f16(42, 1, k * n, 0.1)
    uw = pkg.synth_f16(42, 2, k * n, 0.1)
    x = pkg.synth_f32(42, 3, k)
    for avx in (1, 0):
        g = orc.gemv_f16(x, gw, k, n, T=1, avx512=avx).astype(np.float64)
        u = orc.gemv_f16(x, uw, k, n, T=1, avx512=avx).astype(np.float64)
        got = orc.fused_gate_up_f16(x, gw, uw, k, n, T=1, avx512=avx)
        assert rel_err(got, g / (1 + np.exp(-g)) * u) <= 1e-6


def test_lm_head_f16_row_dot_order(orc, pkg):
    """lm_head_parallel_f16 (gemv.rs:805-822): per row, sum += x[j] * f32(w[j])
    left to right (scalar multiply, then add)."""
    vocab, hidden = 300, 96
    w = pkg.synth_f16(43, 1, vocab * hidden, 0.02)
    x = pkg.synth_f32(43, 2, hidden)
    wf = w.view(np.float16).astype(F32).reshape(vocab, hidden)
    want = np.zeros(vocab, F32)
    for j in range(hidden):
        want = want + F32(x[j]) * wf[:, j]
    assert np.array_equal(orc.lm_head_f16(x, w, vocab, hidden).view(np.uint32), want.view(np.uint32))
    truth = wf.astype(np.float64) @ x.astype(np.float64)
    assert rel_err(orc.lm_head_f16(x, w, vocab, hidden), truth) <= 1e-6


# ---------------------------------------------------------------------------
# RMSNorm, RoPE, softmax, attention, argmax
# ---------------------------------------------------------------------------

def test_rms_norm_order_and_closed_form(orc, pkg):
    """rms_norm_f16 (gemv.rs:744-753): left-fold sum of squares, inv =
    1/sqrt(ss/n + 1e-6), out = x * inv * gamma (eps is 1e-6, hard-coded)."""
    n = 257
    x = pkg.synth_f32(16, 1, n)
    gamma = pkg.synth_f16(16, 2, n, 1.0)
    ss = F32(0)
    for v in x:
        ss = F32(ss + F32(v * v))
    inv = F32(F32(1) / np.sqrt(F32(ss / F32(n)) + F32(1e-6), dtype=F32))
    want = (x * inv).astype(F32) * gamma.view(np.float16).astype(F32)
    assert np.array_equal(orc.rms_norm(x, gamma), want)
    c = 0.75
    got = orc.rms_norm(np.full(64, c, F32), np.full(64, 0x3C00, np.uint16))
    assert np.allclose(got, c / np.sqrt(c * c + 1e-6), rtol=2e-7, atol=0)


def test_rope_identity_norm_and_float64(orc):
    """apply_rope_raw (gemv.rs:757-778): split-half rotation by the table row of `position`."""
    heads, hd, half, pos = 3, 16, 8, 5
    r = rng(17)
    ang = r.uniform(0, 6.3, size=(pos + 1, half))
    cos_t = np.cos(ang).astype(F32).reshape(-1)
    sin_t = np.sin(ang).astype(F32).reshape(-1)
    cos_t[:half] = 1.0                              # position 0: identity row
    sin_t[:half] = 0.0
    data = r.normal(size=heads * hd).astype(F32)
    assert np.array_equal(orc.apply_rope(data, heads, hd, cos_t, sin_t, half, 0), data)
    got = orc.apply_rope(data, heads, hd, cos_t, sin_t, half, pos).reshape(heads, hd)
    d = data.reshape(heads, hd).astype(np.float64)
    c = cos_t[pos * half:(pos + 1) * half].astype(np.float64)
    s = sin_t[pos * half:(pos + 1) * half].astype(np.float64)
    want = np.concatenate([d[:, :half] * c - d[:, half:] * s, d[:, half:] * c + d[:, :half] * s], axis=1)
    assert rel_err(got, want) <= 1e-6
    pair_in = d[:, :half] ** 2 + d[:, half:] ** 2
    pair_out = got[:, :half].astype(np.float64) ** 2 + got[:, half:].astype(np.float64) ** 2
    assert np.allclose(pair_in, pair_out, rtol=1e-5)


def test_softmax_uniform_and_float64(orc):
    """softmax_raw (gemv.rs:782-793); expf is the platform's (parity unpinned bit-wise)."""
    assert np.allclose(orc.softmax(np.full(7, 3.25, F32)), 1 / 7, rtol=1e-6)
    s = rng(18).normal(size=50).astype(F32) * 4
    e = np.exp(s.astype(np.float64) - s.max())
    assert rel_err(orc.softmax(s), e / e.sum()) <= 1e-6


def attention_f64(q, kc, vc, L, H, KVH, hd):
    G = H // KVH
    out = np.zeros((H, hd))
    k = kc.reshape(-1, KVH, hd)[:L].astype(np.float64)
    v = vc.reshape(-1, KVH, hd)[:L].astype(np.float64)
    for h in range(H):
        sc = k[:, h // G] @ q.reshape(H, hd)[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ v[:, h // G]
    return out.reshape(-1)


def test_attention_closed_forms_and_float64(orc):
    """Decode attention (gemv.rs:914-989): head h reads KV head h / groups."""
    H, KVH, hd = 4, 2, 16
    r = rng(19)
    q = r.normal(size=H * hd).astype(F32)
    kc = r.normal(size=(9, KVH, hd)).astype(F32)
    vc = r.normal(size=(9, KVH, hd)).astype(F32)
    one = orc.attention_decode(q, kc, vc, 1, H, KVH, hd).reshape(H, hd)
    for h in range(H):
        assert np.array_equal(one[h], vc[0, h // 2])           # L = 1: output is V
    same_k = np.repeat(kc[:1], 9, axis=0)
    got = orc.attention_decode(q, same_k, vc, 9, H, KVH, hd).reshape(H, hd)
    for h in range(H):                                          # identical keys: mean of V
        assert np.allclose(got[h], vc[:, h // 2].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)
    assert rel_err(orc.attention_decode(q, kc, vc, 9, H, KVH, hd), attention_f64(q, kc, vc, 9, H, KVH, hd)) <= 1e-5


def test_argmax_first_max_rules(orc):
    """sample_token_top_k, temperature <= 0 (generate.rs:346-352): strict >,
    lowest index wins ties, NaN never wins, all -inf/NaN gives index 0."""
    assert orc.argmax(np.array([1, 3, 3, 2], F32)) == 1
    assert orc.argmax(np.array([np.nan, 1, np.nan, 0.5], F32)) == 1
    assert orc.argmax(np.array([-np.inf, -np.inf], F32)) == 0
    assert orc.argmax(np.array([np.nan, np.nan], F32)) == 0
    assert orc.argmax(np.array([-5, np.inf, np.inf], F32)) == 1


# ---------------------------------------------------------------------------
# the full model: composition against a float64 restatement
# ---------------------------------------------------------------------------

def tiny_model(pkg, fmt=1):
    cfg = pkg.ModelConfig(num_layers=2, vocab=50, hidden=64, intermediate=96, num_heads=4, num_kv_heads=2,
                          head_dim=16, rope_half_dim=8, rope_theta=5e6, rope_positions=32)
    w = pkg.synthetic_model(cfg, seed=7, fmt=fmt, rope_positions=32)
    w.no_rope_layers = np.array([0, 1], np.uint8)
    # non-trivial norms so the gamma placement is pinned too
    w.input_norm = [pkg.synth_f16(7, 3000 + l, cfg.hidden, 0.5) for l in range(2)]
    w.post_attn_norm = [pkg.synth_f16(7, 3100 + l, cfg.hidden, 0.5) for l in range(2)]
    w.final_norm = pkg.synth_f16(7, 3200, cfg.hidden, 0.5)
    # the synthetic weights are ~0.02 scale: scale them up so the layers
    # actually change the residual stream
    for ws in w.layers:
        for wt in ws:
            if fmt == 1:
                wt.scales = (wt.scales.view(np.float16).astype(np.float32) * 20).astype(np.float16).view(np.uint16)
            else:
                wt.data = (wt.data.view(np.float16).astype(np.float32) * 20).astype(np.float16).view(np.uint16)
    return w


@pytest.mark.parametrize("fmt,T,avx512", [(1, 1, 1), (0, 1, 1), (0, 1, 0), (0, 3, 1)])
def test_model_decode_and_prefill_vs_float64(orc, pkg, fmt, T, avx512):
    """forward_decode_raw and raw_prefill of the oracle, Q4 and F16 (F16:
    gemv_f16 in both dispatch orders, the two-GEMV gate/up fallback of
    gemv.rs:395-407, the F16 embedding row of gemv.rs:515-526 and
    lm_head_parallel_f16) against the float64 model."""
    w = tiny_model(pkg, fmt)
    f64 = F64Model(w)
    om = orc.OracleModel(w, kv_capacity=32, T=T, avx512=avx512)
    toks = [3, 17, 42, 8, 29]
    for pos, t in enumerate(toks):
        ref = f64.step(t)
        got = om.forward_decode(t)
        assert rel_err(got, ref) <= 1e-4, pos
        assert np.std(ref) > 1e-3                    # the model does something
    for l in range(w.config.num_layers):
        k, v = om.kv_layer(l)
        kr, vr = f64.kv_layer(l)
        assert rel_err(np.ravel(k), np.ravel(kr)) <= 1e-4
        assert rel_err(np.ravel(v), np.ravel(vr)) <= 1e-4
    # raw_prefill (its own GEMM order, gemv.rs:1027-1190) lands on the same state
    om2 = orc.OracleModel(w, kv_capacity=32, T=T, avx512=avx512)
    logits = om2.prefill(toks)
    assert rel_err(logits, ref) <= 1e-4
    for l in range(w.config.num_layers):
        assert rel_err(np.ravel(om2.kv_layer(l)[0]), np.ravel(om.kv_layer(l)[0])) <= 1e-5


def test_model_f16_embedding_row_is_exact(orc, pkg):
    """embed_lookup, F16 arm (gemv.rs:515-522): the row is widened exactly.
    With every projection weight zero the layers add exact zeros to the
    residual, so the logits are lm_head_f16(rms_norm(row)) bit for bit (both
    pinned on their own above)."""
    w = tiny_model(pkg, 0)
    for ws in w.layers:
        for wt in ws:
            wt.data = np.zeros_like(wt.data)
    om = orc.OracleModel(w, kv_capacity=32, T=1)
    tok = 23
    row = w.embed.data.reshape(w.config.vocab, w.config.hidden)[tok].view(np.float16).astype(np.float32)
    want = orc.lm_head_f16(orc.rms_norm(row, w.final_norm), w.embed.data, w.config.vocab, w.config.hidden)
    assert np.array_equal(om.forward_decode(tok), want)


def test_model_greedy_is_argmax_chain(orc, pkg):
    w = tiny_model(pkg)
    om = orc.OracleModel(w, kv_capacity=32, T=1)
    toks, gaps = om.greedy([1, 2, 3], 6)
    om2 = orc.OracleModel(w, kv_capacity=32, T=1)
    logits = om2.prefill([1, 2, 3])
    chain = []
    for _ in range(6):
        t = orc.argmax(logits)
        chain.append(t)
        logits = om2.forward_decode(t)
    assert toks == chain
    assert len(gaps) == 6


def test_kv_set_resumes_like_the_built_cache(orc, pkg):
    """oq_kv_set (a caller-built RawKvCache, gemv.rs:154-166): a cache set
    from another model's rows continues exactly like that model."""
    w = tiny_model(pkg)
    a = orc.OracleModel(w, kv_capacity=32, T=1)
    a.prefill([4, 9, 33, 2])
    b = orc.OracleModel(w, kv_capacity=32, T=1)
    for l in range(w.config.num_layers):
        b.kv_set(l, *a.kv_layer(l))
    assert b.kv_len() == 4
    assert np.array_equal(a.forward_decode(11), b.forward_decode(11))


def test_thread_count_does_not_change_results(orc, pkg):
    """oq_set_threads only spreads independent items (heads, lm_head rows,
    k-split partials) over threads; the partials are added in thread order."""
    k, n = 2048, 2048
    packed, scales = pkg.synth_q4(44, 1, k, n)
    x = pkg.synth_f32(44, 2, k)
    w = tiny_model(pkg)
    outs = []
    for nt in (1, 4):
        orc.set_threads(nt)
        om = orc.OracleModel(w, kv_capacity=32, T=3)
        outs.append((orc.gemv_q4(x, packed, scales, k, n, T=12), om.prefill([1, 5, 7]), om.forward_decode(3)))
    orc.set_threads(0)
    for u, v in zip(*outs):
        assert np.array_equal(u, v)
