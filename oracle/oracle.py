"""ctypes view of the CPU oracle (oracle/myos_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check and by the
bench's CPU-baseline leg, never by the product package. The oracle restates
the reference's CPU path (crates/tensor_core, crates/model_core) bit-for-bit;
see the header of myos_oracle.h for what pins each function.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libmyos_oracle.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
SZ = C.c_size_t


class Shape(C.Structure):
    _fields_ = [
        ("hidden", SZ), ("num_q_heads", SZ), ("num_kv_heads", SZ), ("head_dim", SZ),
        ("intermediate", SZ), ("vocab", SZ), ("num_layers", SZ),
        ("rms_eps", C.c_float), ("rope_theta", C.c_float),
    ]


LAYER_FIELDS = ["ln1", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "ln2", "wg", "wu", "wd"]


class Layer(C.Structure):
    _fields_ = [(f, P) for f in LAYER_FIELDS]


def _declare(L):
    L.orc_bf16_to_f32.argtypes = [C.c_uint16]
    L.orc_bf16_to_f32.restype = C.c_float
    L.orc_gemv_bf16.argtypes = [P, P, P, SZ, SZ]
    L.orc_gemv_bf16_mt.argtypes = [P, P, P, SZ, SZ, C.c_int]
    L.orc_gemm_bf16_mt.argtypes = [P, P, P, SZ, SZ, SZ, C.c_int]
    L.orc_add_bf16_bias.argtypes = [P, P, SZ]
    L.orc_add_bf16_bias.restype = None
    L.orc_embed_gather_bf16.argtypes = [P, P, SZ, SZ, C.c_uint32]
    L.orc_rmsnorm_bf16_weight.argtypes = [P, P, P, SZ, C.c_float]
    L.orc_rope_inv_freqs.argtypes = [P, SZ, C.c_float]
    L.orc_rope_f32_inplace.argtypes = [P, SZ, C.c_uint32, SZ, C.c_float]
    L.orc_attn_scale_f32.argtypes = [SZ]
    L.orc_attn_scale_f32.restype = C.c_float
    L.orc_gqa_attn_f32.argtypes = [P, P, P, P, P, SZ, SZ, SZ, SZ, C.c_int, SZ]
    L.orc_silu_f32.argtypes = [C.c_float]
    L.orc_silu_f32.restype = C.c_float
    L.orc_swiglu_mul_f32.argtypes = [P, P, P, SZ]
    L.orc_swiglu_mul_f32.restype = None
    L.orc_greedy_token.argtypes = [P, SZ]
    L.orc_greedy_token.restype = C.c_uint32
    L.orc_model_new.argtypes = [C.POINTER(Shape), SZ, C.POINTER(Layer), P, P, P, C.c_int]
    L.orc_model_new.restype = P
    L.orc_model_free.argtypes = [P]
    L.orc_model_free.restype = None
    L.orc_forward_token.argtypes = [P, C.c_uint32, SZ]
    L.orc_prefill.argtypes = [P, P, SZ]
    L.orc_greedy_decode.argtypes = [P, SZ, P]
    L.orc_cache_len.argtypes = [P]
    L.orc_cache_len.restype = SZ
    for f in ("orc_logits", "orc_hidden", "orc_normed"):
        getattr(L, f).argtypes = [P]
        getattr(L, f).restype = C.POINTER(C.c_float)
    L.orc_kv_read.argtypes = [P, SZ, SZ, SZ, P, P]
    L.orc_set_threads.argtypes = [P, C.c_int]
    L.orc_set_threads.restype = None
    L.orc_attention_layer.argtypes = [P, SZ, SZ, P, P]
    L.orc_kv_advance.argtypes = [P]
    L.orc_set_kv_bf16.argtypes = [P, C.c_int]
    L.orc_round_bf16.argtypes = [C.c_float]
    L.orc_round_bf16.restype = C.c_float


def _p(a: np.ndarray):
    return a.ctypes.data_as(P)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def bf16_bits_exact(values) -> np.ndarray:
    """f32 values whose low 16 bits are zero -> their bf16 bit patterns."""
    b = f32(values).view(np.uint32)
    assert np.all(b & 0xFFFF == 0), "value not exact in bf16"
    return (b >> 16).astype(np.uint16)


def round_bf16(x) -> np.float32:
    """The value a bf16 KV-cache slot holds for f32 x (nearest, ties to even)."""
    return np.float32(lib().orc_round_bf16(np.float32(x)))


def bf16_to_f32(bits) -> np.ndarray:
    return (u16(bits).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- ops ----

def gemv_bf16(w_bits, x, m, k, threads=0):
    y = np.zeros(m, np.float32)
    w_bits, x = u16(w_bits), f32(x)
    if threads:
        lib().orc_gemv_bf16_mt(_p(y), _p(w_bits), _p(x), m, k, threads)
    else:
        lib().orc_gemv_bf16(_p(y), _p(w_bits), _p(x), m, k)
    return y


def gemm_bf16(w_bits, x, batch, m, k, threads=1):
    y = np.zeros((batch, m), np.float32)
    w_bits, x = u16(w_bits), f32(x)
    lib().orc_gemm_bf16_mt(_p(y), _p(w_bits), _p(x), batch, m, k, threads)
    return y


def add_bf16_bias(y, bias_bits):
    y = f32(y).copy()
    lib().orc_add_bf16_bias(_p(y), _p(u16(bias_bits)), y.size)
    return y


def embed_gather_bf16(table_bits, vocab, hidden, token):
    out = np.zeros(hidden, np.float32)
    rc = lib().orc_embed_gather_bf16(_p(out), _p(u16(table_bits)), vocab, hidden, token)
    return rc, out


def rmsnorm_bf16_weight(gamma_bits, x, eps):
    x = f32(x)
    y = np.zeros_like(x)
    rc = lib().orc_rmsnorm_bf16_weight(_p(y), _p(u16(gamma_bits)), _p(x), x.size, eps)
    assert rc == 0
    return y


def rope_inv_freqs(head_dim, theta):
    t = np.zeros(head_dim // 2, np.float32)
    assert lib().orc_rope_inv_freqs(_p(t), head_dim, theta) == 0
    return t


def rope_f32_inplace(x, position, head_dim, theta):
    x = f32(x).copy()
    rc = lib().orc_rope_f32_inplace(_p(x), x.size, position, head_dim, theta)
    return rc, x


def attn_scale_f32(head_dim):
    return np.float32(lib().orc_attn_scale_f32(head_dim))


def gqa_attn_f32(q, k, v, nq, nkv, head_dim, seq, causal_pos=None):
    q, k, v = f32(q), f32(k), f32(v)
    y = np.zeros(nq * head_dim, np.float32)
    probs = np.zeros(seq, np.float32)
    mask = 0 if causal_pos is None else 1
    rc = lib().orc_gqa_attn_f32(_p(y), _p(q), _p(k), _p(v), _p(probs), nq, nkv, head_dim,
                                seq, mask, 0 if causal_pos is None else causal_pos)
    assert rc == 0
    return y, probs


def silu_f32(z):
    return np.float32(lib().orc_silu_f32(z))


def swiglu_mul_f32(gate, up):
    gate, up = f32(gate), f32(up)
    h = np.zeros_like(gate)
    lib().orc_swiglu_mul_f32(_p(h), _p(gate), _p(up), gate.size)
    return h


def greedy_token(logits):
    logits = f32(logits)
    return int(lib().orc_greedy_token(_p(logits), logits.size))


# -------------------------------------------------------------- model ----

class Model:
    """Oracle model over a dict of BF16 bit arrays keyed by qwen25_layout names."""

    def __init__(self, shape: dict, tensors: dict, max_seq: int, threads: int = 8,
                 kv_bf16: bool = False):
        self._keep = []
        self.shape = dict(shape)
        s = Shape(**{k: shape[k] for k, _ in Shape._fields_})
        n = shape["num_layers"]
        layers = (Layer * n)()
        names = {
            "ln1": "input_layernorm.weight", "wq": "self_attn.q_proj.weight",
            "bq": "self_attn.q_proj.bias", "wk": "self_attn.k_proj.weight",
            "bk": "self_attn.k_proj.bias", "wv": "self_attn.v_proj.weight",
            "bv": "self_attn.v_proj.bias", "wo": "self_attn.o_proj.weight",
            "ln2": "post_attention_layernorm.weight", "wg": "mlp.gate_proj.weight",
            "wu": "mlp.up_proj.weight", "wd": "mlp.down_proj.weight",
        }
        for i in range(n):
            for f, suffix in names.items():
                a = u16(tensors[f"model.layers.{i}.{suffix}"])
                self._keep.append(a)
                setattr(layers[i], f, a.ctypes.data)
        embed = u16(tensors["model.embed_tokens.weight"])
        norm = u16(tensors["model.norm.weight"])
        head = tensors.get("lm_head.weight")
        head = None if head is None else u16(head)
        self._keep += [embed, norm, head, layers]
        self.max_seq = max_seq
        self.h = lib().orc_model_new(C.byref(s), max_seq, layers, embed.ctypes.data,
                                     norm.ctypes.data,
                                     None if head is None else head.ctypes.data, threads)
        if not self.h:
            raise ValueError("oracle rejected the shape")
        if kv_bf16:
            assert lib().orc_set_kv_bf16(self.h, 1) == 0

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_free(self.h)
            self.h = None

    def set_threads(self, t):
        lib().orc_set_threads(self.h, t)

    def forward_token(self, token, pos):
        return lib().orc_forward_token(self.h, token, pos)

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        return lib().orc_prefill(self.h, _p(t), t.size)

    def greedy_decode(self, steps):
        out = np.zeros(steps, np.uint32)
        rc = lib().orc_greedy_decode(self.h, steps, _p(out))
        return rc, out

    def cache_len(self):
        return lib().orc_cache_len(self.h)

    def logits(self):
        return np.ctypeslib.as_array(lib().orc_logits(self.h), (self.shape["vocab"],)).copy()

    def hidden(self):
        return np.ctypeslib.as_array(lib().orc_hidden(self.h), (self.shape["hidden"],)).copy()

    def normed(self):
        return np.ctypeslib.as_array(lib().orc_normed(self.h), (self.shape["hidden"],)).copy()

    def attention_layer(self, layer, pos, residual, proj_in):
        r = f32(residual).copy()
        rc = lib().orc_attention_layer(self.h, layer, pos, _p(r), _p(f32(proj_in)))
        return rc, r

    def advance(self):
        return lib().orc_kv_advance(self.h)

    def kv(self, layer, head, pos):
        d = self.shape["head_dim"]
        k = np.zeros(d, np.float32)
        v = np.zeros(d, np.float32)
        rc = lib().orc_kv_read(self.h, layer, head, pos, _p(k), _p(v))
        assert rc == 0
        return k, v


def load_safetensors_bits(path: str) -> dict:
    """Memory-map a BF16 SafeTensors file: {name: uint16 array (view into the map)}."""
    raw = np.memmap(path, dtype=np.uint8, mode="r")
    n = int(np.frombuffer(raw[:8].tobytes(), "<u8")[0])
    header = json.loads(raw[8:8 + n].tobytes())
    base = 8 + n
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        assert info["dtype"] == "BF16", name
        s, e = info["data_offsets"]
        out[name] = raw[base + s:base + e].view(np.uint16).reshape(info["shape"])
    return out
