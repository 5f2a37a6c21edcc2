"""MI355X (gfx950) batch-1 decode path for QORA's SmolLM3-3B engine.

Python host mirror of the reference crate's model API (src/gemv.rs,
src/save.rs, src/generate.rs) over the C ABI in include/qora_hip.h
(libqora_hip.so, built in-tree by ``make`` in this directory). Everything
that computes runs in the HIP library; this module only moves host buffers
and names things the way the reference does. There is no CPU fallback: if
the library or a GPU is missing, the calls raise.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqora_hip.so")

QORA_HIP_OK = 0
QORA_HIP_E_INVALID = -1
QORA_HIP_E_DEVICE = -2
QORA_HIP_E_NOMEM = -3
QORA_HIP_E_STATE = -4
QORA_HIP_E_IO = -5
QORA_HIP_E_RANGE = -6

FORMAT_F16 = 0
FORMAT_Q4 = 1
KV_F32 = 0
KV_F16 = 1

# Every symbol include/qora_hip.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t


class ModelDesc(ctypes.Structure):
    """qora_model_desc (include/qora_hip.h)."""

    _fields_ = [
        ("num_layers", _U32), ("vocab", _U32), ("hidden", _U32), ("intermediate", _U32),
        ("num_heads", _U32), ("num_kv_heads", _U32), ("head_dim", _U32), ("num_kv_groups", _U32),
        ("rope_half_dim", _U32), ("format", _U32),
        ("layer_wids", _P), ("input_norm", _P), ("post_attn_norm", _P),
        ("embed_wid", _U32), ("final_norm", _P), ("rope_cos", _P), ("rope_sin", _P),
        ("rope_positions", _U64), ("use_rope", _P), ("kv_capacity", _U32), ("kv_dtype", _U32),
    ]


class HostModel(ctypes.Structure):
    """qora_host_model (include/qora_hip.h)."""

    _fields_ = [
        ("num_layers", _U32), ("vocab", _U32), ("hidden", _U32), ("intermediate", _U32),
        ("num_heads", _U32), ("num_kv_heads", _U32), ("head_dim", _U32), ("num_kv_groups", _U32),
        ("rope_half_dim", _U32), ("format", _U32),
        ("w_data", _P), ("w_scales", _P), ("input_norm", _P), ("post_attn_norm", _P),
        ("embed_data", _P), ("embed_scales", _P), ("final_norm", _P),
        ("rope_cos", _P), ("rope_sin", _P), ("rope_positions", _U64), ("use_rope", _P),
    ]


SIGNATURES = {
    "qora_hip_create": (_I, [_I, ctypes.POINTER(_P)]),
    "qora_hip_destroy": (_I, [_P]),
    "qora_hip_last_error": (ctypes.c_char_p, [_P]),
    "qora_hip_device_cus": (_I, [_P]),
    "qora_hip_upload_q4": (_I, [_P, _P, _SZ, _P, _SZ, _U64, _U64, ctypes.POINTER(_U32)]),
    "qora_hip_upload_f16": (_I, [_P, _P, _SZ, _U64, _U64, ctypes.POINTER(_U32)]),
    "qora_hip_weight_ptrs": (_I, [_P, _U32, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "qora_hip_release_weight": (_I, [_P, _U32]),
    "qora_hip_model_init": (_I, [_P, ctypes.POINTER(ModelDesc)]),
    "qora_hip_load_model": (_I, [_P, ctypes.c_char_p, _U32, _U32]),
    "qora_hip_prefill": (_I, [_P, _P, _SZ, _P, ctypes.POINTER(_U32)]),
    "qora_hip_decode": (_I, [_P, _U32, _P, ctypes.POINTER(_U32)]),
    "qora_hip_generate_greedy": (_I, [_P, _U32, _U32, _P]),
    "qora_hip_kv_len": (_I, [_P, ctypes.POINTER(_U64)]),
    "qora_hip_kv_reset": (_I, [_P]),
    "qora_hip_kv_download": (_I, [_P, _U32, _P, _P]),
    "qora_hip_kv_upload": (_I, [_P, _U32, _P, _P, _U64]),
    "qora_hip_malloc": (_I, [_P, _SZ, ctypes.POINTER(_P)]),
    "qora_hip_free": (_I, [_P, _P]),
    "qora_hip_memcpy_h2d": (_I, [_P, _P, _P, _SZ]),
    "qora_hip_memcpy_d2h": (_I, [_P, _P, _P, _SZ]),
    "qora_hip_synchronize": (_I, [_P]),
    "qora_hip_stream": (_P, [_P]),
    "qora_hip_capture_begin": (_I, [_P]),
    "qora_hip_capture_end": (_I, [_P, ctypes.POINTER(_P)]),
    "qora_hip_graph_launch": (_I, [_P, _P, _U32]),
    "qora_hip_graph_destroy": (_I, [_P, _P]),
    "qora_hip_gemv_q4": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_gemv_q4_noalloc": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_gemv_f16": (_I, [_P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_gemv_q4_accumulate": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_gate_up_q4_accumulate": (_I, [_P, _P, _P, _P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_acc_to_f32": (_I, [_P, _P, _U64, _I, _P, _P]),
    "qora_hip_gemv_prepare": (_I, [_P, _U32, _U32, _I, _P]),
    "qora_hip_gemv_run": (_I, [_P, _U32, _P, _P, _P]),
    "qora_hip_gemv_release": (_I, [_P, _U32]),
    "qora_hip_attn_o_limit": (_U32, [_P]),
    "qora_hip_attn_chunk_limit": (_U32, [_P]),
    "qora_hip_lm_head_prepare": (_I, [_P, _U32, _P]),
    "qora_hip_lm_head_run": (_I, [_P, _U32, _P, _P, _P, _P]),
    "qora_hip_gemv_q4_rowdot": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_gemv_f16_rowdot": (_I, [_P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_gate_up_q4": (_I, [_P, _P, _P, _P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_gate_up_f16": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _P]),
    "qora_hip_dequant_q4": (_I, [_P, _P, _P, _U64, _U64, _P, _P]),
    "qora_hip_rmsnorm": (_I, [_P, _P, _P, _U64, _P, _P]),
    "qora_hip_rope": (_I, [_P, _P, _U32, _U32, _P, _P, _U32, _U32, _P]),
    "qora_hip_attn_decode": (_I, [_P, _P, _P, _P, _I, _U32, _U32, _U32, _U32, _P, _P]),
    "qora_hip_gemm": (_I, [_P, _U32, _P, _P, _U64, _P]),
    "qora_hip_attn_prefill": (_I, [_P, _P, _P, _P, _I, _U32, _U32, _U32, _U32, _U32, _P, _P]),
    "qora_hip_sample": (_I, [_P, _P, _U64, _P, _U64, _P, _P, _P, _P]),
    "qora_hip_decode_sample": (_I, [_P, _U32, _P, _U64, _P, _P, _P, _P]),
    "qora_hip_argmax": (_I, [_P, _P, _U64, _P, _P]),
    "qora_synth_q4": (None, [_U64, _U64, _U64, _U64, _P, _P]),
    "qora_synth_f16": (None, [_U64, _U64, _U64, _F, _P]),
    "qora_synth_f32": (None, [_U64, _U64, _U64, _P]),
    "qora_synth_tokens": (None, [_U64, _U64, _U64, _U32, _P]),
    "qora_rope_tables": (None, [_U64, _U32, ctypes.c_double, _P, _P]),
    "qora_file_write": (_I, [ctypes.c_char_p, ctypes.POINTER(HostModel)]),
}

_lib_handle: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libqora_hip.so (built in-tree); raises if it is not built."""
    global _lib_handle
    if _lib_handle is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C qora-llm_amd)")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib_handle = h
    return _lib_handle


class QoraHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"qora_hip error {code}: {msg}")
        self.code = code


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------------------
# synthetic inputs (host, no GPU)
# ---------------------------------------------------------------------------

def synth_q4(seed: int, tensor_id: int, k: int, n: int):
    """Q4 weight [k][n] in the reference layout: (packed u8[k*n/2], scales u16[k*n/32])."""
    packed = np.empty(k * n // 2, dtype=np.uint8)
    scales = np.empty(k * n // 32, dtype=np.uint16)
    lib().qora_synth_q4(seed, tensor_id, k, n, _ptr(packed), _ptr(scales))
    return packed, scales


def synth_f16(seed: int, tensor_id: int, count: int, std: float) -> np.ndarray:
    out = np.empty(count, dtype=np.uint16)
    lib().qora_synth_f16(seed, tensor_id, count, std, _ptr(out))
    return out


def synth_f32(seed: int, tensor_id: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().qora_synth_f32(seed, tensor_id, count, _ptr(out))
    return out


def synth_tokens(seed: int, tensor_id: int, count: int, vocab: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint32)
    lib().qora_synth_tokens(seed, tensor_id, count, vocab, _ptr(out))
    return out


def rope_tables(positions: int, half_dim: int, theta: float):
    cos_t = np.empty(positions * half_dim, dtype=np.float32)
    sin_t = np.empty(positions * half_dim, dtype=np.float32)
    lib().qora_rope_tables(positions, half_dim, theta, _ptr(cos_t), _ptr(sin_t))
    return cos_t, sin_t


# ---------------------------------------------------------------------------
# host model (DecodeWeights, gemv.rs:195-338)
# ---------------------------------------------------------------------------

WEIGHT_NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass
class ModelConfig:
    """Architecture constants of a .qora model (save.rs:173-177, 251-254)."""

    num_layers: int = 36
    vocab: int = 128256
    hidden: int = 2048
    intermediate: int = 11008
    num_heads: int = 16
    num_kv_heads: int = 4
    head_dim: int = 128
    rope_half_dim: int = 64
    rope_theta: float = 5e6
    rope_positions: int = 65536

    @property
    def num_kv_groups(self) -> int:
        return self.num_heads // self.num_kv_heads

    def weight_shapes(self):
        qd = self.num_heads * self.head_dim
        kvd = self.num_kv_heads * self.head_dim
        h, i = self.hidden, self.intermediate
        return [(h, qd), (h, kvd), (h, kvd), (qd, h), (h, i), (h, i), (i, h)]


SMOLLM3_3B = ModelConfig()


@dataclass
class Weight:
    """WeightData (gemv.rs:99-102): Q4 {packed, scales} or F16 {data}, shape k x n."""

    k: int
    n: int
    packed: Optional[np.ndarray] = None   # u8[k*n/2]
    scales: Optional[np.ndarray] = None   # u16[k*n/32]
    data: Optional[np.ndarray] = None     # u16[k*n] (F16)

    @property
    def is_q4(self) -> bool:
        return self.packed is not None

    def memory_bytes(self) -> int:
        return self.packed.nbytes + self.scales.nbytes if self.is_q4 else self.data.nbytes


@dataclass
class DecodeWeights:
    """Host-side mirror of DecodeWeights (gemv.rs:195-206)."""

    config: ModelConfig
    format_id: int                      # 0 = F16, 1 = Q4
    layers: List[List[Weight]]          # [num_layers][7] in WEIGHT_NAMES order
    input_norm: List[np.ndarray]        # u16[hidden]
    post_attn_norm: List[np.ndarray]
    embed: Weight                       # k = vocab, n = hidden
    final_norm: np.ndarray
    rope_cos: np.ndarray                # f32[positions*half]
    rope_sin: np.ndarray
    no_rope_layers: np.ndarray          # u8[num_layers]; 1 = apply RoPE (gemv.rs:885)

    def format_name(self) -> str:
        return {0: "F16", 1: "Q4"}.get(self.format_id, "unknown")

    def num_layers(self) -> int:
        return self.config.num_layers

    def vocab(self) -> int:
        return self.config.vocab

    def hidden(self) -> int:
        return self.config.hidden

    def memory_bytes(self) -> int:
        """DecodeWeights::memory_bytes (gemv.rs:210-226)."""
        t = 0
        for l in range(self.config.num_layers):
            t += sum(w.memory_bytes() for w in self.layers[l])
            t += self.input_norm[l].nbytes + self.post_attn_norm[l].nbytes
        t += self.embed.memory_bytes() + self.final_norm.nbytes
        t += self.rope_cos.nbytes + self.rope_sin.nbytes
        return t

    def weight_bytes_per_token(self) -> int:
        """Bytes of projection + lm_head weights one decode token streams."""
        return sum(w.memory_bytes() for ws in self.layers for w in ws) + self.embed.memory_bytes()


def synthetic_model(config: ModelConfig = SMOLLM3_3B, seed: int = 0, fmt: int = FORMAT_Q4,
                    rope_positions: Optional[int] = None) -> DecodeWeights:
    """Random-init model of `config` from the seeded generator.

    Tensor ids: layer l weight j -> 16*l + j; embedding 1000. Q4 values are
    U{-7..7} with f16 scales |N(0,0.02)|/7; F16 weights N(0, 0.02); norms 1.0;
    RoPE theta from the config on layers 3, 7, ... (i % 4 == 3)."""
    layers = []
    for l in range(config.num_layers):
        ws = []
        for j, (k, n) in enumerate(config.weight_shapes()):
            if fmt == FORMAT_Q4:
                p, s = synth_q4(seed, 16 * l + j, k, n)
                ws.append(Weight(k, n, packed=p, scales=s))
            else:
                ws.append(Weight(k, n, data=synth_f16(seed, 16 * l + j, k * n, 0.02)))
        layers.append(ws)
    if fmt == FORMAT_Q4:
        p, s = synth_q4(seed, 1000, config.vocab, config.hidden)
        embed = Weight(config.vocab, config.hidden, packed=p, scales=s)
    else:
        embed = Weight(config.vocab, config.hidden, data=synth_f16(seed, 1000, config.vocab * config.hidden, 0.02))
    ones = np.full(config.hidden, 0x3C00, dtype=np.uint16)
    positions = rope_positions if rope_positions is not None else config.rope_positions
    cos_t, sin_t = rope_tables(positions, config.rope_half_dim, config.rope_theta)
    flags = np.array([1 if (i % 4 == 3) else 0 for i in range(config.num_layers)], dtype=np.uint8)
    return DecodeWeights(config, fmt, layers, [ones.copy() for _ in range(config.num_layers)],
                         [ones.copy() for _ in range(config.num_layers)], embed, ones.copy(), cos_t, sin_t, flags)


def save_model(weights: DecodeWeights, path: str) -> None:
    """save::save_model (save.rs:119-151) through the C ABI writer."""
    c = weights.config
    keep = []

    def arr(ptrs):
        a = (ctypes.c_void_p * len(ptrs))(*ptrs)
        keep.append(a)
        return ctypes.cast(a, ctypes.c_void_p).value

    w_data = [(_ptr(w.packed) if w.is_q4 else _ptr(w.data)) for ws in weights.layers for w in ws]
    w_scales = [(_ptr(w.scales) if w.is_q4 else 0) for ws in weights.layers for w in ws]
    hm = HostModel(c.num_layers, c.vocab, c.hidden, c.intermediate, c.num_heads, c.num_kv_heads, c.head_dim,
                   c.num_kv_groups, c.rope_half_dim, weights.format_id,
                   arr(w_data), arr(w_scales) if weights.format_id == FORMAT_Q4 else None,
                   arr([_ptr(g) for g in weights.input_norm]), arr([_ptr(g) for g in weights.post_attn_norm]),
                   _ptr(weights.embed.packed) if weights.embed.is_q4 else _ptr(weights.embed.data),
                   _ptr(weights.embed.scales) if weights.embed.is_q4 else None,
                   _ptr(weights.final_norm), _ptr(weights.rope_cos), _ptr(weights.rope_sin),
                   weights.rope_cos.size // c.rope_half_dim, _ptr(weights.no_rope_layers))
    rc = lib().qora_file_write(path.encode(), ctypes.byref(hm))
    if rc != QORA_HIP_OK:
        raise QoraHipError(rc, f"writing {path}")


# ---------------------------------------------------------------------------
# device context and backend
# ---------------------------------------------------------------------------

class HipContext:
    """One qora_hip_ctx: a device, a stream and the buffers it owns."""

    def __init__(self, device: int = 0):
        self.lib = lib()
        h = ctypes.c_void_p()
        rc = self.lib.qora_hip_create(device, ctypes.byref(h))
        if rc != QORA_HIP_OK:
            raise QoraHipError(rc, f"qora_hip_create(device={device}) failed (no usable HIP device?)")
        self.h = h.value

    def check(self, rc: int, what: str = "") -> None:
        if rc != QORA_HIP_OK:
            msg = self.lib.qora_hip_last_error(self.h)
            raise QoraHipError(rc, f"{what}: {msg.decode() if msg else ''}")

    def close(self) -> None:
        if self.h:
            self.lib.qora_hip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def cus(self) -> int:
        return self.lib.qora_hip_device_cus(self.h)

    @property
    def stream(self) -> int:
        return self.lib.qora_hip_stream(self.h)

    # -- memory ------------------------------------------------------------
    def malloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        self.check(self.lib.qora_hip_malloc(self.h, nbytes, ctypes.byref(p)), "malloc")
        return p.value

    def free(self, dptr: int) -> None:
        self.check(self.lib.qora_hip_free(self.h, dptr), "free")

    def to_device(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        d = self.malloc(max(a.nbytes, 16))
        self.check(self.lib.qora_hip_memcpy_h2d(self.h, d, _ptr(a), a.nbytes), "h2d")
        return d

    def h2d(self, dptr: int, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        self.check(self.lib.qora_hip_memcpy_h2d(self.h, dptr, _ptr(a), a.nbytes), "h2d")

    def from_device(self, dptr: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self.check(self.lib.qora_hip_memcpy_d2h(self.h, _ptr(out), dptr, out.nbytes), "d2h")
        return out

    def synchronize(self) -> None:
        self.check(self.lib.qora_hip_synchronize(self.h), "synchronize")

    # -- weights -----------------------------------------------------------
    def upload(self, w: Weight) -> int:
        wid = ctypes.c_uint32()
        if w.is_q4:
            rc = self.lib.qora_hip_upload_q4(self.h, _ptr(w.packed), w.packed.size, _ptr(w.scales), w.scales.size,
                                             w.k, w.n, ctypes.byref(wid))
        else:
            rc = self.lib.qora_hip_upload_f16(self.h, _ptr(w.data), w.data.size, w.k, w.n, ctypes.byref(wid))
        self.check(rc, "upload")
        return wid.value

    def gemv_prepare(self, wid: int, wid_up: int = 0, paired: bool = False) -> int:
        """Packs uploaded weights into the decode step's GEMV tile layout."""
        gid = ctypes.c_uint32()
        self.check(self.lib.qora_hip_gemv_prepare(self.h, wid, wid_up, int(paired), ctypes.byref(gid)),
                   "gemv_prepare")
        return gid.value

    def gemv_run(self, gemv_id: int, x_dev: int, acc_dev: int, stream: int = 0) -> None:
        """acc += x . W (fixed point) with the decode step's GEMV kernel."""
        self.check(self.lib.qora_hip_gemv_run(self.h, gemv_id, x_dev, acc_dev, stream or None), "gemv_run")

    def gemv_release(self, gemv_id: int) -> None:
        self.check(self.lib.qora_hip_gemv_release(self.h, gemv_id), "gemv_release")

    def lm_head_prepare(self, wid: int) -> int:
        """Packs an uploaded Q4 [rows][cols] weight into the lm_head tile layout."""
        lid = ctypes.c_uint32()
        self.check(self.lib.qora_hip_lm_head_prepare(self.h, wid, ctypes.byref(lid)), "lm_head_prepare")
        return lid.value

    def lm_head_run(self, lm_id: int, x_dev: int, logits_dev: int, argmax_dev: int = 0, stream: int = 0) -> None:
        """logits = W . x with the decode step's lm_head kernel; argmax_dev (device
        int32) receives the greedy token when given."""
        self.check(self.lib.qora_hip_lm_head_run(self.h, lm_id, x_dev, logits_dev, argmax_dev or None,
                                                 stream or None), "lm_head_run")

    def sample(self, logits_dev: int, vocab: int, history: Sequence[int], params: "SampleParams",
               rng_state: int):
        """Penalties and top-k/top-p sampling of device logits; returns (token, new rng state)."""
        hist = np.ascontiguousarray(np.asarray(history, dtype=np.uint32))
        st = ctypes.c_uint64(rng_state)
        tok = ctypes.c_uint32()
        self.check(self.lib.qora_hip_sample(self.h, logits_dev, vocab, _ptr(hist) if hist.size else None, hist.size,
                                            ctypes.byref(params), ctypes.byref(st), ctypes.byref(tok), None),
                   "sample")
        return tok.value, st.value

    def weight_ptrs(self, wid: int):
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        self.check(self.lib.qora_hip_weight_ptrs(self.h, wid, ctypes.byref(a), ctypes.byref(b)), "weight_ptrs")
        return a.value, b.value

    # -- graphs ------------------------------------------------------------
    def capture_begin(self) -> None:
        self.check(self.lib.qora_hip_capture_begin(self.h), "capture_begin")

    def capture_end(self) -> int:
        g = ctypes.c_void_p()
        self.check(self.lib.qora_hip_capture_end(self.h, ctypes.byref(g)), "capture_end")
        return g.value

    def graph_launch(self, g: int, count: int = 1) -> None:
        self.check(self.lib.qora_hip_graph_launch(self.h, g, count), "graph_launch")

    def graph_destroy(self, g: int) -> None:
        self.check(self.lib.qora_hip_graph_destroy(self.h, g), "graph_destroy")


class SampleParams(ctypes.Structure):
    """qora_sample_params: GenerateParams' sampling fields (generate.rs:15-35)."""

    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("repetition_penalty", ctypes.c_float), ("presence_penalty", ctypes.c_float)]


# main.rs:130-141 defaults
DEFAULT_SAMPLING = dict(temperature=0.7, top_p=0.95, top_k=20, repetition_penalty=1.1, presence_penalty=1.5)


class HipBackend:
    """The device-resident model: forward_decode_raw / raw_prefill on the GPU.

    Mirrors the reference's decode API (gemv.rs:872-876, 1027-1030) with the
    RawKvCache held on the device inside the context."""

    def __init__(self, ctx: HipContext, weights: DecodeWeights, kv_capacity: int = 2048, kv_dtype: int = KV_F32,
                 shared_layers: bool = False):
        """shared_layers: every layer uses layer 0's uploaded weights (one layer's
        bytes on the device: a cache-residency probe, not a model)."""
        self.ctx = ctx
        self.weights = weights
        c = weights.config
        self.config = c
        self.kv_capacity = kv_capacity
        self.kv_dtype = kv_dtype
        if shared_layers:
            wids = np.array([ctx.upload(w) for w in weights.layers[0]] * c.num_layers, dtype=np.uint32)
        else:
            wids = np.array([ctx.upload(w) for ws in weights.layers for w in ws], dtype=np.uint32)
        embed_wid = ctx.upload(weights.embed)
        self._keep = [wids]
        in_ptrs = (ctypes.c_void_p * c.num_layers)(*[_ptr(g) for g in weights.input_norm])
        post_ptrs = (ctypes.c_void_p * c.num_layers)(*[_ptr(g) for g in weights.post_attn_norm])
        self._keep += [in_ptrs, post_ptrs]
        d = ModelDesc(c.num_layers, c.vocab, c.hidden, c.intermediate, c.num_heads, c.num_kv_heads, c.head_dim,
                      c.num_kv_groups, c.rope_half_dim, weights.format_id, _ptr(wids),
                      ctypes.cast(in_ptrs, ctypes.c_void_p).value, ctypes.cast(post_ptrs, ctypes.c_void_p).value,
                      embed_wid, _ptr(weights.final_norm), _ptr(weights.rope_cos), _ptr(weights.rope_sin),
                      weights.rope_cos.size // c.rope_half_dim, _ptr(weights.no_rope_layers), kv_capacity, kv_dtype)
        self._desc = d
        self.model_init()
        self.wids = wids.reshape(c.num_layers, 7)
        self.embed_wid = embed_wid

    def model_init(self) -> None:
        """(Re)builds the device model from the uploaded weights
        (qora_hip_model_init); the KV cache starts empty."""
        self.ctx.check(self.ctx.lib.qora_hip_model_init(self.ctx.h, ctypes.byref(self._desc)), "model_init")

    def forward_decode_raw(self, token_id: int, want_logits: bool = True):
        """One decode step; returns (logits or None, greedy token)."""
        logits = np.empty(self.config.vocab, dtype=np.float32) if want_logits else None
        tok = ctypes.c_uint32()
        self.ctx.check(self.ctx.lib.qora_hip_decode(self.ctx.h, int(token_id), _ptr(logits) if want_logits else None,
                                                    ctypes.byref(tok)), "decode")
        return logits, tok.value

    def raw_prefill(self, token_ids: Sequence[int], want_logits: bool = True):
        ids = np.ascontiguousarray(np.asarray(token_ids, dtype=np.uint32))
        logits = np.empty(self.config.vocab, dtype=np.float32) if want_logits else None
        tok = ctypes.c_uint32()
        self.ctx.check(self.ctx.lib.qora_hip_prefill(self.ctx.h, _ptr(ids), ids.size,
                                                     _ptr(logits) if want_logits else None, ctypes.byref(tok)),
                       "prefill")
        return logits, tok.value

    def generate_greedy(self, token_id: int, steps: int) -> np.ndarray:
        out = np.empty(max(steps, 1), dtype=np.uint32)
        self.ctx.check(self.ctx.lib.qora_hip_generate_greedy(self.ctx.h, int(token_id), steps, _ptr(out)),
                       "generate_greedy")
        return out[:steps]

    def kv_len(self) -> int:
        n = ctypes.c_uint64()
        self.ctx.check(self.ctx.lib.qora_hip_kv_len(self.ctx.h, ctypes.byref(n)), "kv_len")
        return n.value

    def kv_reset(self) -> None:
        self.ctx.check(self.ctx.lib.qora_hip_kv_reset(self.ctx.h), "kv_reset")

    def attn_o_limit(self) -> int:
        """Steps appending a position below this run attention inside the o GEMV."""
        return int(self.ctx.lib.qora_hip_attn_o_limit(self.ctx.h))

    def attn_chunk_limit(self) -> int:
        """Steps appending a position from attn_o_limit() up to below this run
        the chunked attention + o step."""
        return int(self.ctx.lib.qora_hip_attn_chunk_limit(self.ctx.h))

    def kv_layer(self, layer: int):
        """(k, v) of one layer as f32 [len][kv_heads*head_dim] (RawKvCache entry)."""
        n = self.kv_len()
        kvd = self.config.num_kv_heads * self.config.head_dim
        k = np.empty((max(n, 1), kvd), dtype=np.float32)
        v = np.empty((max(n, 1), kvd), dtype=np.float32)
        self.ctx.check(self.ctx.lib.qora_hip_kv_download(self.ctx.h, layer, _ptr(k), _ptr(v)), "kv_download")
        return k[:n], v[:n]

    def decode_sample(self, token_id: int, history: Sequence[int], params: "SampleParams", rng_state: int,
                      want_logits: bool = False):
        """One decode step, then the penalties and top-k/top-p sampling on the
        device; returns (logits or None, token, new rng state)."""
        hist = np.ascontiguousarray(np.asarray(history, dtype=np.uint32))
        logits = np.empty(self.config.vocab, dtype=np.float32) if want_logits else None
        st = ctypes.c_uint64(rng_state)
        tok = ctypes.c_uint32()
        self.ctx.check(self.ctx.lib.qora_hip_decode_sample(self.ctx.h, int(token_id), _ptr(hist) if hist.size else None,
                                                           hist.size, ctypes.byref(params), ctypes.byref(st),
                                                           _ptr(logits) if want_logits else None, ctypes.byref(tok)),
                       "decode_sample")
        return logits, tok.value, st.value

    def kv_upload(self, layer: int, k: np.ndarray, v: np.ndarray) -> None:
        """Sets one layer's cache rows [0, len) from f32 [len][kv_heads*head_dim]
        and the cache length to len."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        if k.shape != v.shape or k.ndim != 2:
            raise ValueError("k and v must be [len][kv_heads*head_dim]")
        self.ctx.check(self.ctx.lib.qora_hip_kv_upload(self.ctx.h, layer, _ptr(k), _ptr(v), k.shape[0]),
                       "kv_upload")


def generate_greedy_host(backend: HipBackend, prompt: Sequence[int], steps: int) -> List[int]:
    """generate_raw (generate.rs:272-342) with temperature 0 and no EOS or
    loop-detection stop: prefill, then feed each argmax back, host-driven."""
    _, tok = backend.raw_prefill(prompt, want_logits=False)
    out = [tok]
    for _ in range(steps - 1):
        _, tok = backend.forward_decode_raw(tok, want_logits=False)
        out.append(tok)
    return out
