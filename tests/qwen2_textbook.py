"""An independent float64 Qwen2 decoder forward, written from the model's
mathematical definition (pre-norm residual blocks; RMSNorm; NeoX rotary
embedding over the pairs (i, i + d/2); grouped-query attention where query
head h reads kv head h // (nq / nkv); SwiGLU MLP down(silu(gate(n)) * up(n));
final RMSNorm and a tied or untied head).

It is vectorised numpy in double precision and shares no code with the
oracle, so it is used to check the oracle's composition (which buffer feeds
which projection, the residual adds, per-layer cache slots, the head) on
small random models. An f32 chain and an f64 evaluation of the same model
differ by rounding only (relative ~1e-6 at these sizes); a wiring mistake
moves results by O(1).
"""
from __future__ import annotations

import numpy as np


def bf16_f64(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32).astype(np.float64)


class Textbook:
    def __init__(self, s: dict, t: dict):
        self.s = s
        H, nq, nkv, d = s["hidden"], s["num_q_heads"], s["num_kv_heads"], s["head_dim"]
        self.eps = float(s["rms_eps"])
        self.theta = float(s["rope_theta"])
        self.embed = bf16_f64(t["model.embed_tokens.weight"]).reshape(s["vocab"], H)
        self.head = (bf16_f64(t["lm_head.weight"]).reshape(s["vocab"], H)
                     if "lm_head.weight" in t else self.embed)
        self.final = bf16_f64(t["model.norm.weight"])
        self.layers = []
        for l in range(s["num_layers"]):
            g = lambda suf: bf16_f64(t[f"model.layers.{l}.{suf}"])
            self.layers.append(dict(
                ln1=g("input_layernorm.weight"), ln2=g("post_attention_layernorm.weight"),
                wq=g("self_attn.q_proj.weight").reshape(nq * d, H),
                bq=g("self_attn.q_proj.bias"),
                wk=g("self_attn.k_proj.weight").reshape(nkv * d, H),
                bk=g("self_attn.k_proj.bias"),
                wv=g("self_attn.v_proj.weight").reshape(nkv * d, H),
                bv=g("self_attn.v_proj.bias"),
                wo=g("self_attn.o_proj.weight").reshape(H, nq * d),
                wg=g("mlp.gate_proj.weight").reshape(s["intermediate"], H),
                wu=g("mlp.up_proj.weight").reshape(s["intermediate"], H),
                wd=g("mlp.down_proj.weight").reshape(H, s["intermediate"])))
        # per layer: lists of rotated keys / values by position
        self.K = [[] for _ in range(s["num_layers"])]
        self.V = [[] for _ in range(s["num_layers"])]

    def _rms(self, x, g):
        return g * (x / np.sqrt(np.mean(x * x) + self.eps))

    def _rope(self, v, pos, heads):
        d = self.s["head_dim"]
        half = d // 2
        inv = self.theta ** (-(2.0 * np.arange(half)) / d)
        c, sn = np.cos(pos * inv), np.sin(pos * inv)
        v = v.reshape(heads, d).copy()
        a, b = v[:, :half].copy(), v[:, half:].copy()
        v[:, :half] = a * c - b * sn
        v[:, half:] = b * c + a * sn
        return v

    def forward(self, token: int):
        """One token at position len(cache); returns (logits, hidden, normed)."""
        s = self.s
        nq, nkv, d = s["num_q_heads"], s["num_kv_heads"], s["head_dim"]
        pos = len(self.K[0])
        x = self.embed[token].copy()
        for l, w in enumerate(self.layers):
            n = self._rms(x, w["ln1"])
            q = self._rope(w["wq"] @ n + w["bq"], pos, nq)
            k = self._rope(w["wk"] @ n + w["bk"], pos, nkv)
            v = (w["wv"] @ n + w["bv"]).reshape(nkv, d)
            self.K[l].append(k)
            self.V[l].append(v)
            K = np.stack(self.K[l], 1)  # [nkv, seq, d]
            V = np.stack(self.V[l], 1)
            att = np.empty((nq, d))
            for h in range(nq):
                g = h // (nq // nkv)
                sc = K[g] @ q[h] / np.sqrt(d)
                p = np.exp(sc - sc.max())
                att[h] = (p / p.sum()) @ V[g]
            x = x + w["wo"] @ att.ravel()
            n2 = self._rms(x, w["ln2"])
            gt, up = w["wg"] @ n2, w["wu"] @ n2
            x = x + w["wd"] @ (gt / (1.0 + np.exp(-gt)) * up)
        normed = self._rms(x, self.final)
        return self.head @ normed, x, normed

    def kv(self, layer, head, pos):
        return self.K[layer][pos][head], self.V[layer][pos][head]
