"""Shared test helpers (inputs, tolerances, device buffers)."""
import contextlib

import numpy as np

# Tolerance of the north-star parity bar for floating-point outputs:
# max_j |gpu_j - ref_j| / max_j |ref_j| <= 1e-3 (fp32 accumulation).
REL_TOL = 1e-3


def rel_err(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    denom = max(float(np.max(np.abs(b))) if b.size else 0.0, 1e-30)
    return float(np.max(np.abs(a - b))) / denom if a.size else 0.0


def elem_err(a, b, mag) -> float:
    """max_j |a_j - b_j| / mag_j, each output's error against its own scale
    mag_j = sum_k |x_k w_kj| (what the rounding error of a sum of products is
    proportional to). Unlike rel_err, which measures every error against the
    largest output, this bounds the small outputs too; an output whose terms
    are all zero (mag_j = 0) must be exact."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    m = np.asarray(mag, dtype=np.float64)
    return float(np.max(np.abs(a - b) / (m + 1e-300))) if a.size else 0.0


def rng(seed):
    return np.random.default_rng(seed)


def random_q4(r, k, n, scale_std=0.02):
    """Random Q4 weight in the reference layout with f16 scales |N(0,std)|/7."""
    q = r.integers(1, 16, size=(k, n), dtype=np.uint8)          # q in [1,15] -> v in [-7,7]
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    scales = (np.abs(r.normal(0, scale_std, size=(k, n // 32))) / 7).astype(np.float16).view(np.uint16).reshape(-1)
    return np.ascontiguousarray(packed), np.ascontiguousarray(scales)


def exact_q4(r, k, n):
    """Q4 weight with power-of-two scales 2^-1..2^-4 (exact-arithmetic regime)."""
    q = r.integers(0, 16, size=(k, n), dtype=np.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    e = r.integers(1, 5, size=(k, n // 32))
    scales = (2.0 ** -e).astype(np.float16).view(np.uint16).reshape(-1)
    return np.ascontiguousarray(packed), np.ascontiguousarray(scales)


def dequant_np(packed, scales, k, n):
    """float64 dequant straight from the layout definition (gemv.rs:7-9, 31-32)."""
    p = packed.reshape(k, n // 2)
    q = np.empty((k, n), dtype=np.int64)
    q[:, 0::2] = p & 0x0F
    q[:, 1::2] = p >> 4
    s = scales.view(np.float16).astype(np.float64).reshape(k, n // 32)
    return (q - 8) * np.repeat(s, 32, axis=1)


class Dev:
    """Device buffers of one test, freed at exit."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.ptrs = []

    def put(self, a):
        p = self.ctx.to_device(np.ascontiguousarray(a))
        self.ptrs.append(p)
        return p

    def empty(self, nbytes):
        p = self.ctx.malloc(max(int(nbytes), 16))
        self.ptrs.append(p)
        return p

    def get(self, p, shape, dtype):
        return self.ctx.from_device(p, shape, dtype)

    def close(self):
        self.ctx.synchronize()
        for p in self.ptrs:
            self.ctx.free(p)
        self.ptrs = []


@contextlib.contextmanager
def device(ctx):
    d = Dev(ctx)
    try:
        yield d
    finally:
        d.close()
