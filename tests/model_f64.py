"""Float64 restatement of the decode and prefill steps from the model's
definition, for Q4 and F16 weights (the truth the oracle and the GPU are
both held to).

forward_decode_raw (gemv.rs:872-1019): embed -> per layer [RMSNorm, q/k/v,
RoPE on flagged layers at the cache length, append K/V, GQA attention, o,
residual, RMSNorm, silu(gate)*up, down, residual] -> final RMSNorm -> tied
lm_head. raw_prefill (gemv.rs:1027-1190) computes the same values token by
token. Every value here is float64; only the stored inputs (nibbles, binary16
scales and weights, f32 RoPE tables) are shared with the code under test."""
import numpy as np

from helpers import dequant_np


def weight_f64(wt):
    """A Q4 or F16 Weight as a float64 [k][n] matrix."""
    if wt.packed is not None:
        return dequant_np(wt.packed, wt.scales, wt.k, wt.n)
    return wt.data.view(np.float16).astype(np.float64).reshape(wt.k, wt.n)


def f16_vec(a):
    return a.view(np.float16).astype(np.float64)


class F64Model:
    def __init__(self, w):
        self.w = w
        self.c = w.config
        self.mats = [[weight_f64(t) for t in ws] for ws in w.layers]
        self.embed = weight_f64(w.embed)
        self.reset()

    def reset(self):
        self.cache = [([], []) for _ in range(self.c.num_layers)]

    def _rms(self, x, g):
        return x / np.sqrt(np.mean(x * x) + 1e-6) * f16_vec(g)

    def _rope(self, v, heads, pos):
        c, w = self.c, self.w
        v = v.reshape(heads, c.head_dim).copy()
        half = c.rope_half_dim
        ct = w.rope_cos[pos * half:(pos + 1) * half].astype(np.float64)
        st = w.rope_sin[pos * half:(pos + 1) * half].astype(np.float64)
        a, b = v[:, :half].copy(), v[:, half:2 * half].copy()
        v[:, :half], v[:, half:2 * half] = a * ct - b * st, b * ct + a * st
        return v.reshape(-1)

    def step(self, token):
        """One forward_decode_raw step; returns the logits (float64)."""
        c, w = self.c, self.w
        pos = len(self.cache[0][0])
        x = self.embed[token].copy()
        for l in range(c.num_layers):
            Wq, Wk, Wv, Wo, Wg, Wu, Wd = self.mats[l]
            xn = self._rms(x, w.input_norm[l])
            q, k, v = xn @ Wq, xn @ Wk, xn @ Wv
            if w.no_rope_layers[l]:
                q, k = self._rope(q, c.num_heads, pos), self._rope(k, c.num_kv_heads, pos)
            self.cache[l][0].append(k)
            self.cache[l][1].append(v)
            K = np.array(self.cache[l][0]).reshape(-1, c.num_kv_heads, c.head_dim)
            V = np.array(self.cache[l][1]).reshape(-1, c.num_kv_heads, c.head_dim)
            att = np.zeros((c.num_heads, c.head_dim))
            for h in range(c.num_heads):
                sc = K[:, h // c.num_kv_groups] @ q.reshape(c.num_heads, c.head_dim)[h] / np.sqrt(c.head_dim)
                p = np.exp(sc - sc.max())
                att[h] = (p / p.sum()) @ V[:, h // c.num_kv_groups]
            x = x + att.reshape(-1) @ Wo
            xn = self._rms(x, w.post_attn_norm[l])
            g, u = xn @ Wg, xn @ Wu
            x = x + (g / (1 + np.exp(-g)) * u) @ Wd
        return self._rms(x, w.final_norm) @ self.embed.T

    def prefill(self, ids):
        self.reset()
        logits = None
        for t in ids:
            logits = self.step(int(t))
        return logits

    def kv_layer(self, layer):
        return np.array(self.cache[layer][0]), np.array(self.cache[layer][1])
