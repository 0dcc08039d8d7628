"""Tiny Qwen2.5-shaped weight maps used by the oracle and GPU tests.

block_fixture / rich_map restate the reference's in-process fixtures
(crates/model_core/src/qwen25_block.rs:788-826 and :1302-1382) as BF16 bit
arrays keyed by the qwen25_layout names (qwen25_layout.rs:102-189).
"""
from __future__ import annotations

import json
import struct

import numpy as np

LAYER_SUFFIXES = [
    "input_layernorm.weight",
    "self_attn.q_proj.weight",
    "self_attn.q_proj.bias",
    "self_attn.k_proj.weight",
    "self_attn.k_proj.bias",
    "self_attn.v_proj.weight",
    "self_attn.v_proj.bias",
    "self_attn.o_proj.weight",
    "post_attention_layernorm.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
]

THETA = np.float32(1e6)


def bits(values, shape=None) -> np.ndarray:
    """Exact-in-bf16 f32 values -> uint16 bf16 bit patterns."""
    a = np.ascontiguousarray(values, dtype=np.float32)
    u = a.view(np.uint32)
    assert np.all(u & 0xFFFF == 0), "fixture value not exact in bf16"
    out = (u >> 16).astype(np.uint16)
    return out.reshape(shape) if shape is not None else out


def rne_bf16(values) -> np.ndarray:
    """Round f32 values to bf16 (round to nearest, ties to even) -> bit patterns."""
    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def shape_dict(hidden, nq, nkv, d, inter, vocab, layers, eps, theta=THETA):
    return dict(hidden=hidden, num_q_heads=nq, num_kv_heads=nkv, head_dim=d,
                intermediate=inter, vocab=vocab, num_layers=layers,
                rms_eps=np.float32(eps), rope_theta=np.float32(theta))


def tensor_shapes(s: dict, tied=True) -> dict:
    H, I, V = s["hidden"], s["intermediate"], s["vocab"]
    qd = s["num_q_heads"] * s["head_dim"]
    kd = s["num_kv_heads"] * s["head_dim"]
    per = [(H,), (qd, H), (qd,), (kd, H), (kd,), (kd, H), (kd,), (H, qd), (H,), (I, H), (I, H),
           (H, I)]
    out = {"model.embed_tokens.weight": (V, H), "model.norm.weight": (H,)}
    for l in range(s["num_layers"]):
        for suf, shp in zip(LAYER_SUFFIXES, per):
            out[f"model.layers.{l}.{suf}"] = shp
    if not tied:
        out["lm_head.weight"] = (V, H)
    return out


# -------------------------------------------------------- block fixture ----

def fixture_shape(layers=1):
    """qwen25_block.rs:788-805: hidden 2, vocab 4, eps 0."""
    return shape_dict(2, 2, 1, 2, 2, 4, layers, 0.0)


def block_fixture_layer(t, layer, q_b, v_b, o_w, gate, up, down):
    """fill_layer, qwen25_block.rs:845-912."""
    p = f"model.layers.{layer}."
    t[p + "input_layernorm.weight"] = bits([1.0, 1.0])
    t[p + "self_attn.q_proj.weight"] = bits(np.zeros(8), (4, 2))
    t[p + "self_attn.q_proj.bias"] = bits(q_b)
    t[p + "self_attn.k_proj.weight"] = bits(np.zeros(4), (2, 2))
    t[p + "self_attn.k_proj.bias"] = bits(np.zeros(2))
    t[p + "self_attn.v_proj.weight"] = bits(np.zeros(4), (2, 2))
    t[p + "self_attn.v_proj.bias"] = bits(v_b)
    t[p + "self_attn.o_proj.weight"] = bits(o_w, (2, 4))
    t[p + "post_attention_layernorm.weight"] = bits([1.0, 1.0])
    t[p + "mlp.gate_proj.weight"] = bits(gate, (2, 2))
    t[p + "mlp.up_proj.weight"] = bits(up, (2, 2))
    t[p + "mlp.down_proj.weight"] = bits(down, (2, 2))


FIXTURE_EMBED = [1.0, 1.0, 2.0, 0.0, 0.0, 4.0, -1.0, 0.0]


def fixture_embed_and_final(final_gamma=(1.0, 0.0)):
    """insert_embed_and_final, qwen25_block.rs:828-840: embed rows [1,1], [2,0],
    [0,4], [-1,0]; final gamma [1, 0]."""
    return {
        "model.embed_tokens.weight": bits(FIXTURE_EMBED, (4, 2)),
        "model.norm.weight": bits(list(final_gamma)),
    }


def block_fixture():
    """block_fixture, qwen25_block.rs:811-826: token 0 -> logits [1, 2, 0, -1]."""
    t = fixture_embed_and_final()
    block_fixture_layer(t, 0, [0.5, 0.0, 0.0, 0.25], [1.0, 0.0],
                        [1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0], [0.0] * 4, [0.0] * 4,
                        [0.0] * 4)
    return fixture_shape(), t


def swiglu_residual_fixture():
    """swiglu_residual_changes_the_logits, qwen25_block.rs:1074-1129: the block
    fixture with gate = up = [[1, 0], [0, 0]] and down = identity, so the MLP
    adds [silu(1), 0] to the stream [2, 2]."""
    t = fixture_embed_and_final()
    block_fixture_layer(t, 0, [0.5, 0.0, 0.0, 0.25], [1.0, 0.0],
                        [1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0],
                        [1.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 1.0])
    return fixture_shape(), t


def two_layer_fixture():
    """two_layers_advance_once_per_token, qwen25_block.rs:1132-1197: o_proj and
    the MLP are zero in both layers; V biases [2, 0] (layer 0) and [0, 8]
    (layer 1), stored at the same cursor."""
    t = fixture_embed_and_final()
    zero_o, zero_mlp = [0.0] * 8, [0.0] * 4
    block_fixture_layer(t, 0, [0.0] * 4, [2.0, 0.0], zero_o, zero_mlp, zero_mlp, zero_mlp)
    block_fixture_layer(t, 1, [0.0] * 4, [0.0, 8.0], zero_o, zero_mlp, zero_mlp, zero_mlp)
    return fixture_shape(2), t


def bf16_kv_fixture():
    """The block fixture's shape with a value projection whose outputs are
    not bf16 values: token 0 normalises to [1, 1], so v = [1 + 3 * 2^-8,
    1 + 2^-9] exactly in f32, and a bf16 cache slot rounds them (nearest,
    ties to even) to [1 + 2^-6, 1]. q = k = 0, so attention weights every
    position equally; o_proj copies head 0's output into the stream and the
    MLP is zero, so the hidden state after the layer is [1, 1] + attention."""
    t = fixture_embed_and_final()
    p = "model.layers.0."
    block_fixture_layer(t, 0, [0.0] * 4, [0.0, 0.0],
                        [1.0, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0], [0.0] * 4, [0.0] * 4,
                        [0.0] * 4)
    t[p + "self_attn.v_proj.weight"] = bits([1.0, 3.0 * 2.0 ** -8, 1.0, 2.0 ** -9], (2, 2))
    return fixture_shape(), t


def bf16_kv_fixture_wide():
    """bf16_kv_fixture widened to a shape the cooperative decode kernels take
    (hidden 64, 2 q heads / 1 kv head of dim 32, intermediate 64, vocab 8,
    eps 0): token 0 embeds to 64 ones, so its norm is exactly 1 and v starts
    [1 + 3 * 2^-8, 1 + 2^-9, 0, ...]; q = k = 0; o_proj copies head 0's
    first two output columns into stream rows 0 and 1; the MLP is zero. The
    hidden state after the layer is 1 + [v0, v1, 0, ...] with v as the cache
    holds it, exactly, in any summation order."""
    s = shape_dict(64, 2, 1, 32, 64, 8, 1, 0.0)
    t = {name: bits(np.zeros(shp, np.float32)) for name, shp in tensor_shapes(s).items()}
    emb = np.zeros((8, 64), np.float32)
    emb[0] = 1.0
    emb[1, :2] = [2.0, -1.0]
    t["model.embed_tokens.weight"] = bits(emb)
    t["model.norm.weight"] = bits(np.ones(64, np.float32))
    p = "model.layers.0."
    for n in ("input_layernorm.weight", "post_attention_layernorm.weight"):
        t[p + n] = bits(np.ones(64, np.float32))
    wv = np.zeros((32, 64), np.float32)
    wv[0, :2] = [1.0, 3.0 * 2.0 ** -8]
    wv[1, :2] = [1.0, 2.0 ** -9]
    t[p + "self_attn.v_proj.weight"] = bits(wv)
    wo = np.zeros((64, 64), np.float32)
    wo[0, 0] = wo[1, 1] = 1.0
    t[p + "self_attn.o_proj.weight"] = bits(wo)
    return s, t


# ------------------------------------------------------------- rich map ----

_PAT = np.array([0.5, -0.25, 1.0, 0.0, -1.0, 0.125, 2.0, -0.5], np.float32)


def _put_pat(shape, salt):
    n = int(np.prod(shape))
    return bits(_PAT[(np.arange(n) + salt) % 8], shape)


def rich_shape(layers=2):
    """The chunk-prefill test shape, qwen25_block.rs:1425-1438."""
    return shape_dict(8, 4, 2, 2, 6, 5, layers, 1e-6)


def rich_map(s: dict):
    """rich_map, qwen25_block.rs:1302-1353 (patterned exact-bf16 weights)."""
    shp = tensor_shapes(s)
    t = {
        "model.embed_tokens.weight": _put_pat(shp["model.embed_tokens.weight"], 1),
        "model.norm.weight": _put_pat(shp["model.norm.weight"], 2),
    }
    for l in range(s["num_layers"]):
        salt = 10 + l * 20
        for j, suf in enumerate(LAYER_SUFFIXES):
            key = f"model.layers.{l}.{suf}"
            t[key] = _put_pat(shp[key], salt + j)
    return t


# ------------------------------------------------------ seeded random ----

def random_map(s: dict, seed: int, std=0.02, tied=True, gains_one=True):
    """Seeded N(0, std) BF16 weights (RNE), norm gains 1.0 when gains_one."""
    rng = np.random.default_rng(seed)
    t = {}
    for name, shp in tensor_shapes(s, tied).items():
        if gains_one and name.endswith("norm.weight"):
            t[name] = bits(np.ones(shp, np.float32))
        else:
            t[name] = rne_bf16(rng.standard_normal(shp, dtype=np.float32) * np.float32(std))
    return t


def write_safetensors(path: str, tensors: dict):
    """Minimal BF16 SafeTensors writer (8-byte LE header length + JSON + payload)."""
    header = {}
    off = 0
    names = sorted(tensors)
    for n in names:
        a = np.ascontiguousarray(tensors[n], dtype=np.uint16)
        header[n] = {"dtype": "BF16", "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for n in names:
            f.write(np.ascontiguousarray(tensors[n], dtype=np.uint16).tobytes())
