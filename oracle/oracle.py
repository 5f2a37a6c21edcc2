"""ctypes wrapper of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP library and the timed CPU
baseline of bench.py. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module. See oracle.h for what pins each
function and which parts stay "parity unpinned".
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I = ctypes.c_int


class OqModelDesc(ctypes.Structure):
    _fields_ = [
        ("num_layers", _U32), ("vocab", _U32), ("hidden", _U32), ("intermediate", _U32),
        ("num_heads", _U32), ("num_kv_heads", _U32), ("head_dim", _U32), ("num_kv_groups", _U32),
        ("rope_half_dim", _U32), ("format", _U32),
        ("w_data", _P), ("w_scales", _P), ("in_norm", _P), ("post_norm", _P),
        ("embed_data", _P), ("embed_scales", _P), ("final_norm", _P),
        ("rope_cos", _P), ("rope_sin", _P), ("use_rope", _P),
    ]


_SIGS = {
    "oq_h2f": (ctypes.c_float, [ctypes.c_uint16]),
    "oq_dequant_q4_row": (None, [_P, _P, _U64, _U64, _P]),
    "oq_dequant_q4": (None, [_P, _P, _U64, _U64, _P]),
    "oq_gemv_q4_rows": (None, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "oq_gemv_q4": (None, [_P, _P, _P, _U64, _U64, _I, _P]),
    "oq_fused_gate_up_q4": (None, [_P, _P, _P, _P, _P, _U64, _U64, _I, _P]),
    "oq_gemv_f16": (None, [_P, _P, _U64, _U64, _I, _I, _P]),
    "oq_fused_gate_up_f16": (None, [_P, _P, _P, _U64, _U64, _I, _I, _P]),
    "oq_lm_head_q4": (None, [_P, _P, _P, _U64, _U64, _P]),
    "oq_lm_head_f16": (None, [_P, _P, _U64, _U64, _P]),
    "oq_rms_norm_f16": (None, [_P, _P, _U64, _P]),
    "oq_apply_rope": (None, [_P, _U64, _U64, _P, _P, _U64, _U64]),
    "oq_softmax": (None, [_P, _U64]),
    "oq_attention_decode": (None, [_P, _P, _P, _U64, _U64, _U64, _U64, _P]),
    "oq_argmax": (_U32, [_P, _U64]),
    "oq_kv_create": (_P, [_U32, _U32, _U64]),
    "oq_kv_free": (None, [_P]),
    "oq_kv_len": (_U64, [_P, _U32]),
    "oq_kv_k": (_P, [_P, _U32]),
    "oq_kv_v": (_P, [_P, _U32]),
    "oq_kv_set": (_I, [_P, _U32, _P, _P, _U64]),
    "oq_rng_next_f32": (ctypes.c_float, [_P]),
    "oq_repetition_penalty": (None, [_P, _U64, _P, _U64, ctypes.c_float]),
    "oq_presence_penalty": (None, [_P, _U64, _P, _U64, ctypes.c_float]),
    "oq_sample_top_k": (_U32, [_P, _U64, ctypes.c_float, ctypes.c_float, _U64, _P]),
    "oq_forward_decode": (_I, [ctypes.POINTER(OqModelDesc), _P, _U32, _I, _I, _P]),
    "oq_prefill": (_I, [ctypes.POINTER(OqModelDesc), _P, _P, _U64, _I, _P]),
    "oq_set_threads": (None, [_I]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (make -C oracle)")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _lib = h
    return _lib


def _p(a):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- kernels -------------------------------------------------------------

def dequant_q4(packed, scales, k, n):
    out = np.empty(k * n, dtype=np.float32)
    lib().oq_dequant_q4(_p(packed), _p(scales), k, n, _p(out))
    return out.reshape(k, n)


def gemv_q4(x, packed, scales, k, n, T=1):
    x = f32(x)
    out = np.empty(n, dtype=np.float32)
    lib().oq_gemv_q4(_p(x), _p(packed), _p(scales), k, n, T, _p(out))
    return out


def gemv_q4_rows(x, packed, scales, n, k0, k1):
    x = f32(x)
    out = np.empty(n, dtype=np.float32)
    lib().oq_gemv_q4_rows(_p(x), _p(packed), _p(scales), n, k0, k1, _p(out))
    return out


def fused_gate_up_q4(x, gp, gs, up, us, k, n, T=1):
    x = f32(x)
    out = np.empty(n, dtype=np.float32)
    lib().oq_fused_gate_up_q4(_p(x), _p(gp), _p(gs), _p(up), _p(us), k, n, T, _p(out))
    return out


def gemv_f16(x, w, k, n, T=1, avx512=1):
    x = f32(x)
    out = np.empty(n, dtype=np.float32)
    lib().oq_gemv_f16(_p(x), _p(w), k, n, T, avx512, _p(out))
    return out


def fused_gate_up_f16(x, gw, uw, k, n, T=1, avx512=1):
    x = f32(x)
    out = np.empty(n, dtype=np.float32)
    lib().oq_fused_gate_up_f16(_p(x), _p(gw), _p(uw), k, n, T, avx512, _p(out))
    return out


def lm_head_q4(x, packed, scales, vocab, hidden):
    x = f32(x)
    out = np.empty(vocab, dtype=np.float32)
    lib().oq_lm_head_q4(_p(x), _p(packed), _p(scales), vocab, hidden, _p(out))
    return out


def lm_head_f16(x, w, vocab, hidden):
    x = f32(x)
    out = np.empty(vocab, dtype=np.float32)
    lib().oq_lm_head_f16(_p(x), _p(w), vocab, hidden, _p(out))
    return out


def rms_norm(x, gamma):
    x = f32(x)
    out = np.empty_like(x)
    lib().oq_rms_norm_f16(_p(x), _p(gamma), x.size, _p(out))
    return out


def apply_rope(data, num_heads, head_dim, cos_t, sin_t, half_dim, position):
    d = f32(data).copy()
    lib().oq_apply_rope(_p(d), num_heads, head_dim, _p(f32(cos_t)), _p(f32(sin_t)), half_dim, position)
    return d


def softmax(scores):
    s = f32(scores).copy()
    lib().oq_softmax(_p(s), s.size)
    return s


def attention_decode(q, kc, vc, L, num_heads, num_kv_heads, head_dim):
    out = np.empty(num_heads * head_dim, dtype=np.float32)
    lib().oq_attention_decode(_p(f32(q)), _p(f32(kc)), _p(f32(vc)), L, num_heads, num_kv_heads, head_dim, _p(out))
    return out


def argmax(logits):
    return int(lib().oq_argmax(_p(f32(logits)), logits.size))


def h2f(h):
    return lib().oq_h2f(int(h))


def set_threads(n):
    lib().oq_set_threads(int(n))


# ---- model -----------------------------------------------------------------

class OracleModel:
    """forward_decode_raw / raw_prefill of the reference on host weights.

    `weights` is a DecodeWeights-like object (config, format_id, layers,
    input_norm, post_attn_norm, embed, final_norm, rope_cos, rope_sin,
    no_rope_layers) holding numpy arrays."""

    def __init__(self, weights, kv_capacity=2048, T=1, avx512=1):
        self.w = weights
        c = weights.config
        self.c = c
        self.T = T
        self.avx512 = avx512
        self.kv_capacity = kv_capacity
        fl = [w for ws in weights.layers for w in ws]
        q4 = weights.format_id == 1
        self._wd = (ctypes.c_void_p * len(fl))(*[_p(w.packed) if q4 else _p(w.data) for w in fl])
        self._ws = (ctypes.c_void_p * len(fl))(*[_p(w.scales) if q4 else None for w in fl])
        self._in = (ctypes.c_void_p * c.num_layers)(*[_p(g) for g in weights.input_norm])
        self._post = (ctypes.c_void_p * c.num_layers)(*[_p(g) for g in weights.post_attn_norm])
        self.desc = OqModelDesc(
            c.num_layers, c.vocab, c.hidden, c.intermediate, c.num_heads, c.num_kv_heads, c.head_dim,
            c.num_kv_groups, c.rope_half_dim, weights.format_id,
            ctypes.cast(self._wd, ctypes.c_void_p).value, ctypes.cast(self._ws, ctypes.c_void_p).value,
            ctypes.cast(self._in, ctypes.c_void_p).value, ctypes.cast(self._post, ctypes.c_void_p).value,
            _p(weights.embed.packed) if q4 else _p(weights.embed.data),
            _p(weights.embed.scales) if q4 else None, _p(weights.final_norm),
            _p(weights.rope_cos), _p(weights.rope_sin), _p(weights.no_rope_layers))
        self.kv = None
        self.reset()

    def reset(self):
        if self.kv:
            lib().oq_kv_free(self.kv)
        self.kv = lib().oq_kv_create(self.c.num_layers, self.c.num_kv_heads * self.c.head_dim, self.kv_capacity)

    def __del__(self):
        try:
            if self.kv:
                lib().oq_kv_free(self.kv)
        except Exception:
            pass

    def forward_decode(self, token):
        logits = np.empty(self.c.vocab, dtype=np.float32)
        rc = lib().oq_forward_decode(ctypes.byref(self.desc), self.kv, int(token), self.T, self.avx512, _p(logits))
        if rc != 0:
            raise RuntimeError("oracle forward_decode failed (cache full or bad token)")
        return logits

    def prefill(self, ids):
        self.reset()
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
        logits = np.empty(self.c.vocab, dtype=np.float32)
        rc = lib().oq_prefill(ctypes.byref(self.desc), self.kv, _p(ids), ids.size, self.T, _p(logits))
        if rc != 0:
            raise RuntimeError("oracle prefill failed")
        return logits

    def kv_len(self, layer=0):
        return int(lib().oq_kv_len(self.kv, layer))

    def kv_layer(self, layer):
        n = self.kv_len(layer)
        kvd = self.c.num_kv_heads * self.c.head_dim
        kp = lib().oq_kv_k(self.kv, layer)
        vp = lib().oq_kv_v(self.kv, layer)
        k = np.ctypeslib.as_array((ctypes.c_float * (n * kvd)).from_address(kp)).reshape(n, kvd).copy()
        v = np.ctypeslib.as_array((ctypes.c_float * (n * kvd)).from_address(vp)).reshape(n, kvd).copy()
        return k, v

    def kv_set(self, layer, k, v):
        """Sets one layer's cache rows [0, len) from f32 [len][kv_heads*head_dim]."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        if lib().oq_kv_set(self.kv, layer, _p(k), _p(v), k.shape[0]) != 0:
            raise RuntimeError("oracle kv_set: bad layer or beyond the capacity")

    def greedy(self, prompt, steps):
        """Prefill then `steps` greedy tokens (generate_raw with temperature 0)."""
        logits = self.prefill(prompt)
        toks = [argmax(logits)]
        gaps = [top2_gap(logits)]
        for _ in range(steps - 1):
            logits = self.forward_decode(toks[-1])
            toks.append(argmax(logits))
            gaps.append(top2_gap(logits))
        return toks, gaps


def rng_next_f32(state):
    """Rng::next_f32 (generate.rs:54-60); returns (value, new state)."""
    st = ctypes.c_uint64(state)
    v = lib().oq_rng_next_f32(ctypes.byref(st))
    return v, st.value


def sample(logits, history, temperature, top_p, top_k, repetition_penalty, presence_penalty, rng_state):
    """apply_repetition_penalty, apply_presence_penalty, sample_token_top_k
    (generate.rs:64-91, 345-395) on a copy; returns (token, new rng state).
    Penalties apply only when sampling (temperature > 0), as at generate.rs:132-136."""
    lg = np.ascontiguousarray(logits, dtype=np.float32).copy()
    h = np.ascontiguousarray(np.asarray(history, dtype=np.uint32))
    if temperature > 0:
        lib().oq_repetition_penalty(_p(lg), lg.size, _p(h), h.size, repetition_penalty)
        lib().oq_presence_penalty(_p(lg), lg.size, _p(h), h.size, presence_penalty)
    st = ctypes.c_uint64(rng_state)
    tok = lib().oq_sample_top_k(_p(lg), lg.size, temperature, top_p, top_k, ctypes.byref(st))
    return int(tok), st.value


def top2_gap(logits):
    """(top1 - top2) of a logits vector, to flag near-ties in greedy parity."""
    part = np.partition(logits, -2)[-2:]
    return float(part[1] - part[0])
