"""Host-side checks that need no GPU: the C ABI library's exports, its error
paths, the seeded synthetic generator, the .qora writer, byte accounting and
the bench's one-GPU contract."""
import ctypes
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qora_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qora_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function(pkg):
    lib = pkg.lib()
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python bindings describe each of them
    assert set(names) <= set(pkg.SIGNATURES), sorted(set(names) - set(pkg.SIGNATURES))


def test_create_forced_failure_returns_error(pkg, monkeypatch):
    """QORA_HIP_FORCE_FAIL=init: qora_hip_create fails cleanly (the host keeps
    the reference's fall-back-to-CPU behaviour, main.rs:143-151)."""
    monkeypatch.setenv("QORA_HIP_FORCE_FAIL", "init")
    lib = pkg.lib()
    h = ctypes.c_void_p()
    rc = lib.qora_hip_create(0, ctypes.byref(h))
    assert rc != pkg.QORA_HIP_OK and not h.value
    with pytest.raises(pkg.QoraHipError):
        pkg.HipContext(0)


def test_null_context_calls_are_rejected(pkg):
    lib = pkg.lib()
    assert lib.qora_hip_destroy(None) == pkg.QORA_HIP_E_INVALID
    assert lib.qora_hip_decode(None, 1, None, None) != pkg.QORA_HIP_OK
    assert lib.qora_hip_gemv_q4(None, None, None, None, None, 1, 32, None) != pkg.QORA_HIP_OK


# ---------------------------------------------------------------------------
# seeded generator (qora_synth_*) against a numpy restatement
# ---------------------------------------------------------------------------

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def mix64(z):
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def stream_key(seed, tid):
    return int(mix64(np.uint64(seed) ^ mix64(np.uint64((tid + 0x632BE59BD9B4E019) & M64))))


def draws(key, count):
    i = np.arange(count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix64(np.uint64(key) + (i + np.uint64(1)) * np.uint64(GOLDEN))


def normals(r):
    """Box-Muller from the two 32-bit halves of each draw; ln by frexp and an
    atanh series, cos by a halved-angle Taylor series, each operation a
    correctly rounded float64 one (so every byte matches the library)."""
    u1 = ((r >> np.uint64(32)).astype(np.float64) + 0.5) * 2.0 ** -32
    u2 = ((r & np.uint64(0xFFFFFFFF)).astype(np.float64) + 0.5) * 2.0 ** -32
    m, e = np.frexp(u1)
    low = m < 0.70710678118654752
    m = np.where(low, m * 2.0, m)
    e = np.where(low, e - 1, e)
    t = (m - 1.0) / (m + 1.0)
    t2 = t * t
    s = np.full_like(t, 1.0 / 23.0)
    for k in range(10, -1, -1):
        s = s * t2 + 1.0 / (2.0 * k + 1.0)
    ln = e.astype(np.float64) * 0.6931471805599453 + 2.0 * t * s
    coef = [1.0]
    for k in range(1, 13):
        coef.append(-coef[-1] / ((2.0 * k - 1.0) * (2.0 * k)))
    h = 0.5 * (6.283185307179586 * (u2 - 0.5))
    h2 = h * h
    c = np.full_like(h, coef[12])
    for k in range(11, -1, -1):
        c = c * h2 + coef[k]
    return np.sqrt(-2.0 * ln) * (2.0 * c * c - 1.0)


def test_normals_restatement_is_gaussian():
    # the series against numpy's log and cos, and the moments of a large sample
    r = draws(stream_key(5, 3), 200000)
    z = normals(r)
    u1 = ((r >> np.uint64(32)).astype(np.float64) + 0.5) * 2.0 ** -32
    u2 = ((r & np.uint64(0xFFFFFFFF)).astype(np.float64) + 0.5) * 2.0 ** -32
    ref = np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * (u2 - 0.5))
    assert np.max(np.abs(z - ref)) < 1e-13
    assert abs(float(np.mean(z))) < 0.01 and abs(float(np.std(z)) - 1.0) < 0.01
    assert abs(float(np.mean(z ** 4)) - 3.0) < 0.05          # Gaussian kurtosis (Irwin-Hall(4) gives 2.7)
    assert 4.0 < float(np.max(np.abs(z))) < 6.8


def test_synth_q4_matches_restatement(pkg):
    k, n = 48, 96
    packed, scales = pkg.synth_q4(3, 21, k, n)
    nbytes = k * n // 2
    r = draws(stream_key(3, 42), (nbytes + 3) // 4)
    want = np.empty(nbytes, np.uint8)
    for m in range(4):
        idx = np.arange(len(r)) * 4 + m
        ok = idx < nbytes
        lo = ((r >> np.uint64(16 * m)) & np.uint64(0xFF)).astype(np.uint32)
        hi = ((r >> np.uint64(16 * m + 8)) & np.uint64(0xFF)).astype(np.uint32)
        q = (((lo * 15) >> 8) + 1) | ((((hi * 15) >> 8) + 1) << 4)
        want[idx[ok]] = q[ok]
    assert np.array_equal(packed, want)
    s = np.abs(normals(draws(stream_key(3, 43), k * n // 32))) * (0.02 / 7.0)
    assert np.array_equal(scales, s.astype(np.float32).astype(np.float16).view(np.uint16))
    q = np.concatenate([packed & 15, packed >> 4])
    assert q.min() >= 1 and q.max() <= 15          # values in [-7, 7]


def test_synth_f16_f32_tokens_match_restatement(pkg):
    v16 = pkg.synth_f16(9, 5, 1000, 0.02)
    assert np.array_equal(v16, (normals(draws(stream_key(9, 10), 1000)) * 0.02).astype(np.float32)
                          .astype(np.float16).view(np.uint16))
    v32 = pkg.synth_f32(9, 6, 1000)
    assert np.array_equal(v32, normals(draws(stream_key(9, 12), 1000)).astype(np.float32))
    toks = pkg.synth_tokens(9, 7, 500, 128256)
    d = draws(stream_key(9, 14), 500)
    assert np.array_equal(toks, (((d >> np.uint64(32)) * np.uint64(128256)) >> np.uint64(32)).astype(np.uint32))
    assert abs(float(np.mean(v32))) < 0.15 and 0.85 < float(np.std(v32)) < 1.15


def test_rope_tables(pkg):
    """cos/sin(pos * theta^(-2i/(2 half))) computed in float64 then rounded;
    the reference loads its tables from the file and ships no generator."""
    cos_t, sin_t = pkg.rope_tables(100, 64, 5e6)
    inv = 5e6 ** (-(2.0 * np.arange(64)) / 128.0)
    a = np.arange(100)[:, None] * inv[None, :]
    assert np.allclose(cos_t.reshape(100, 64), np.cos(a), rtol=0, atol=6e-8)
    assert np.allclose(sin_t.reshape(100, 64), np.sin(a), rtol=0, atol=6e-8)
    assert np.all(cos_t[:64] == 1.0) and np.all(sin_t[:64] == 0.0)


# ---------------------------------------------------------------------------
# .qora writer against an independent parser of the format (save.rs)
# ---------------------------------------------------------------------------

class QoraReader:
    def __init__(self, data):
        self.d, self.o = data, 0

    def take(self, n):
        b = self.d[self.o:self.o + n]
        assert len(b) == n, "truncated"
        self.o += n
        return b

    def u8(self):
        return self.take(1)[0]

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def vec(self, dtype):
        n = self.u64()
        return np.frombuffer(self.take(n * np.dtype(dtype).itemsize), dtype=dtype)


def parse_qora(path):
    r = QoraReader(open(path, "rb").read())
    assert r.take(4) == b"QOR3" and r.u32() == 1
    fmt = r.u8()
    L, vocab, hidden, half = r.u32(), r.u32(), r.u32(), r.u32()
    flags = r.vec(np.uint8)

    def weight():
        k, n = r.u64(), r.u64()
        if fmt == 1:
            return k, n, r.vec(np.uint8), r.vec(np.uint16)
        return k, n, r.vec(np.uint16), None

    layers = []
    for _ in range(L):
        ws = [weight() for _ in range(7)]
        g1, g2 = r.vec(np.uint16), r.vec(np.uint16)
        heads = (r.u32(), r.u32(), r.u32(), r.u32())
        layers.append((ws, g1, g2, heads))
    embed = weight()
    final = r.vec(np.uint16)
    cos_t, sin_t = r.vec(np.float32), r.vec(np.float32)
    assert r.o == len(r.d)
    return dict(fmt=fmt, L=L, vocab=vocab, hidden=hidden, half=half, flags=flags, layers=layers, embed=embed,
                final=final, cos=cos_t, sin=sin_t)


@pytest.mark.parametrize("fmt", [1, 0])
def test_qora_writer_matches_format(pkg, tmp_path, fmt):
    import __graft_entry__ as entry
    cfg = entry.smoke_config(pkg)
    cfg.num_layers = 2
    w = pkg.synthetic_model(cfg, seed=4, fmt=fmt, rope_positions=16)
    path = str(tmp_path / "m.qora")
    pkg.save_model(w, path)
    f = parse_qora(path)
    assert (f["fmt"], f["L"], f["vocab"], f["hidden"], f["half"]) == (fmt, 2, cfg.vocab, cfg.hidden,
                                                                      cfg.rope_half_dim)
    assert np.array_equal(f["flags"], w.no_rope_layers)
    for l in range(2):
        ws, g1, g2, heads = f["layers"][l]
        assert heads == (cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.num_kv_groups)
        assert np.array_equal(g1, w.input_norm[l]) and np.array_equal(g2, w.post_attn_norm[l])
        for j, (k, n, a, b) in enumerate(ws):
            wt = w.layers[l][j]
            assert (k, n) == (wt.k, wt.n)
            if fmt == 1:
                assert np.array_equal(a, wt.packed) and np.array_equal(b, wt.scales)
            else:
                assert np.array_equal(a, wt.data)
    assert np.array_equal(f["final"], w.final_norm)
    assert np.array_equal(f["cos"], w.rope_cos) and np.array_equal(f["sin"], w.rope_sin)


# ---------------------------------------------------------------------------
# byte accounting and the bench contract
# ---------------------------------------------------------------------------

def test_smollm3_q4_bytes_per_token(pkg):
    """1,729,658,880 B of Q4 weights stream per decode token (36 layers of
    q, k, v, o, gate, up, down plus the tied 128256 x 2048 lm_head); the
    gate projection alone is 12,681,216 B."""
    c = pkg.SMOLLM3_3B
    q4 = lambda k, n: k * n // 2 + k * n // 16
    per_layer = sum(q4(k, n) for k, n in c.weight_shapes())
    assert q4(2048, 11008) == 12_681_216
    assert c.num_layers * per_layer + q4(c.vocab, c.hidden) == 1_729_658_880


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stdout


def _header_params():
    """{function: parameter count} of include/qora_hip.h."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(qora_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def _header_struct_fields(name):
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct \{([^}]*)\}\s*" + name + r"\s*;", text).group(1)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if decl:
            head, *rest = [p.strip() for p in decl.split(",")]
            fields.append(re.findall(r"(\w+)\s*$", head)[0])
            fields.extend(rest)
    return fields


def test_rust_binding_matches_the_header():
    """qora-llm_amd/rust/qora-hip-sys/src/lib.rs (the FFI crate a Rust host links)
    declares every header function with the same number of arguments, and its
    #[repr(C)] structs have the header's fields in the header's order."""
    src = open(os.path.join(ROOT, "qora-llm_amd", "rust", "qora-hip-sys", "src", "lib.rs")).read()
    src = re.sub(r"//[^\n]*", "", src)
    rust = {}
    for name, args in re.findall(r"pub fn (qora_[a-z0-9_]+)\s*\(([^)]*)\)", src):
        args = args.strip().rstrip(",")
        rust[name] = 0 if not args else args.count(",") + 1
    want = _header_params()
    assert set(rust) == set(want), (sorted(set(want) - set(rust)), sorted(set(rust) - set(want)))
    assert {n: rust[n] for n in want if rust[n] != want[n]} == {}
    for struct in ("qora_model_desc", "qora_sample_params", "qora_host_model"):
        body = re.search(r"pub struct " + struct + r"\s*\{([^}]*)\}", src).group(1)
        rfields = re.findall(r"pub (\w+)\s*:", body)
        assert rfields == _header_struct_fields(struct), struct
