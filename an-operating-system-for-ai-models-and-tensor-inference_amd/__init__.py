"""MI355X (gfx950) implementation of the batch-1 BF16-weight / FP32-accumulate
token loop, exposed with the reference's operator names.

Op tier (crates/tensor_core/src/lib.rs:54-74): gemv_bf16, gemm_bf16,
add_bf16_bias, embed_gather_bf16, rmsnorm_bf16_weight, rope_f32_inplace,
gqa_attn_f32, swiglu_mul_f32, greedy_token -- on torch tensors that live on
the GPU (torch only provides device memory and the stream). Model tier
(crates/model_core/src/lib.rs:21-26): Model.open / prefill / forward_token /
greedy_decode over a BF16 SafeTensors file.

Errors are raised as MyosError whose `.kind` names the reference's variant
(Shape, TokenOutOfBounds, RowOutOfBounds, Position, Full, Range, Missing,
DType, ...); as in the reference, a failed call leaves its outputs and the
KV cursor untouched. Every call goes through libmyos_hip.so; if it is not
built this package raises on import of the library, there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "_build", "libmyos_hip.so")
CLI_PATH = os.path.join(PKG_DIR, "_build", "myos")
INCLUDE = os.path.join(os.path.dirname(PKG_DIR), "include", "myos_hip.h")

OK, E_SHAPE, E_TOKEN, E_ROW_OOB, E_POSITION, E_KV_FULL, E_KV_RANGE = range(7)
E_W_MISSING, E_W_DTYPE, E_W_SHAPE, E_W_LENGTH, E_IO, E_PARSE, E_HIP, E_ARG = range(7, 15)
E_SCRATCH = 15

KIND = {
    E_SHAPE: "Shape", E_TOKEN: "TokenOutOfBounds", E_ROW_OOB: "RowOutOfBounds",
    E_POSITION: "Position", E_KV_FULL: "Full", E_KV_RANGE: "Range", E_W_MISSING: "Missing",
    E_W_DTYPE: "DType", E_W_SHAPE: "WeightShape", E_W_LENGTH: "Length", E_IO: "Io",
    E_PARSE: "Parse", E_HIP: "Hip", E_ARG: "Arg", E_SCRATCH: "Scratch",
}

KV_F32, KV_BF16 = 0, 1
DECODE_AUTO, DECODE_KERNELS, DECODE_PERSISTENT, DECODE_STREAMED = 0, 1, 2, 3
SHAPE_QWEN25_1_5B, SHAPE_QWEN25_7B = 0, 1


class MyosError(RuntimeError):
    def __init__(self, code: int, what: str = ""):
        self.code = code
        self.kind = KIND.get(code, f"status{code}")
        super().__init__(f"{what}: {self.kind} ({_strerror(code)})")


_lib = None
P, SZ, F32, U32, I32 = C.c_void_p, C.c_size_t, C.c_float, C.c_uint32, C.c_int


class BlockShape(C.Structure):
    """BlockShape + AttnShape (qwen25_block.rs:53-75, attn_wire.rs:44-63)."""
    _fields_ = [("hidden", SZ), ("num_q_heads", SZ), ("num_kv_heads", SZ), ("head_dim", SZ),
                ("intermediate", SZ), ("vocab", SZ), ("num_layers", SZ), ("rms_eps", F32),
                ("rope_theta", F32), ("tied_head", I32)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


EXPORTS = {
    "myos_strerror": ([I32], C.c_char_p),
    "myos_build_info": ([], C.c_char_p),
    "myos_gemv_bf16": ([P, SZ, P, SZ, P, SZ, SZ, SZ, P], I32),
    "myos_gemm_bf16": ([P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, P], I32),
    "myos_gemm_bf16_noalloc": ([P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, P], I32),
    "myos_gemm_bf16_noalloc_scratch": ([SZ, SZ, SZ], SZ),
    "myos_gemm_bf16_noalloc_max_scratch": ([], SZ),
    "myos_add_bf16_bias": ([P, SZ, P, SZ, P], I32),
    "myos_embed_gather_bf16": ([P, SZ, P, SZ, SZ, SZ, U32, P], I32),
    "myos_rmsnorm_bf16_weight": ([P, SZ, P, SZ, P, SZ, F32, P], I32),
    "myos_rope_f32_inplace": ([P, SZ, U32, SZ, F32, P], I32),
    "myos_gqa_attn_f32": ([P, SZ, P, SZ, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, I32, SZ, P], I32),
    "myos_swiglu_mul_f32": ([P, SZ, P, SZ, P, SZ, P], I32),
    "myos_swiglu_bf16": ([P, SZ, P, SZ, P, SZ, P, SZ, P, SZ, P, SZ, P, SZ, P, SZ, SZ, SZ, P], I32),
    "myos_silu_f32": ([P, SZ, P, SZ, P], I32),
    "myos_rmsnorm_f32": ([P, SZ, P, SZ, P, SZ, F32, P], I32),
    "myos_rope_inv_freqs": ([P, SZ, SZ, F32, P], I32),
    "myos_attn_scale_f32": ([SZ, C.POINTER(F32)], I32),
    "myos_greedy_token": ([P, P, SZ, P], I32),
    "myos_stream_sync": ([P], I32),
    "myos_block_shape_preset": ([I32, C.POINTER(BlockShape)], I32),
    "myos_model_open": ([C.c_char_p, C.POINTER(BlockShape), I32, SZ, C.POINTER(P)], I32),
    "myos_model_close": ([P], None),
    "myos_prefill": ([P, P, SZ], I32),
    "myos_forward_token": ([P, U32, SZ], I32),
    "myos_greedy_decode": ([P, SZ, P], I32),
    "myos_cache_len": ([P], SZ),
    "myos_attention_layer": ([P, SZ, SZ, P, P, SZ], I32),
    "myos_kv_advance": ([P], I32),
    "myos_max_seq": ([P], SZ),
    "myos_copy_logits": ([P, P, SZ], I32),
    "myos_copy_hidden": ([P, P, SZ], I32),
    "myos_copy_normed": ([P, P, SZ], I32),
    "myos_kv_read": ([P, SZ, SZ, SZ, P, P], I32),
    "myos_set_graph": ([P, I32], I32),
    "myos_set_decode_mode": ([P, I32], I32),
    "myos_decode_path": ([P], I32),
    "myos_set_decode_trace": ([P, C.c_int64], I32),
    "myos_copy_decode_trace": ([P, P, SZ], I32),
    "myos_debug_raise_wait_error": ([P], I32),
    "myos_decode_forced": ([P, P, SZ, P], I32),
    "myos_last_prefill_ms": ([P], C.c_double),
    "myos_last_decode_ms": ([P], C.c_double),
    "myos_weight_bytes": ([P], SZ),
    "myos_kv_bytes": ([P], SZ),
    "myos_write_random_qwen25": ([C.c_char_p, C.POINTER(BlockShape), C.c_uint64, F32, I32], I32),
    "myos_cache_clear": ([P], I32),
    "myos_sha256_file": ([C.c_char_p, C.c_char_p], I32),
    "myos_time_kernel": ([P, I32, I32, C.POINTER(C.c_double)], I32),
    "myos_kernel_bytes": ([P, I32], C.c_double),
}

K_QKV, K_ATTN, K_O, K_GATE_UP, K_DOWN, K_HEAD = range(6)
KERNEL_NAMES = ["qkv_rope_kv", "attn_decode", "o_resid", "gate_up_swiglu", "down_resid",
                "lm_head_argmax"]


def lib():
    """Load libmyos_hip.so (built by build.py); raises if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                              f"python {os.path.join(PKG_DIR, 'build.py')}")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in EXPORTS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _strerror(code: int) -> str:
    try:
        return lib().myos_strerror(code).decode()
    except Exception:  # the library may be what failed to load
        return "?"


def _check(code: int, what: str):
    if code != OK:
        raise MyosError(code, what)


def build_info() -> str:
    return lib().myos_build_info().decode()


def preset(which: int = SHAPE_QWEN25_1_5B) -> BlockShape:
    s = BlockShape()
    _check(lib().myos_block_shape_preset(which, C.byref(s)), "preset")
    return s


def make_shape(hidden, num_q_heads, num_kv_heads, head_dim, intermediate, vocab, num_layers,
               rms_eps=1e-6, rope_theta=1e6, tied_head=True) -> BlockShape:
    return BlockShape(hidden, num_q_heads, num_kv_heads, head_dim, intermediate, vocab,
                      num_layers, rms_eps, rope_theta, 1 if tied_head else 0)


# ---------------------------------------------------------------- op tier ----

def _dev(t, name):
    """(pointer, element count) of a contiguous GPU tensor."""
    if t is None:
        return None, 0
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return C.c_void_p(t.data_ptr()), t.numel()


def _w16(t, name):
    import torch
    if t.dtype not in (torch.bfloat16, torch.int16, torch.uint16):
        raise ValueError(f"{name} must hold BF16 bit patterns (bfloat16/int16/uint16)")
    return _dev(t, name)


def _f32(t, name):
    import torch
    if t.dtype != torch.float32:
        raise ValueError(f"{name} must be float32")
    return _dev(t, name)


def _stream(stream):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def gemv_bf16(y, w, x, m, k, stream=None):
    """bf16.rs:80-122: y[m] = W[m, k] x[k] (f32 accumulate)."""
    yp, yn = _f32(y, "y")
    wp, wn = _w16(w, "w")
    xp, xn = _f32(x, "x")
    _check(lib().myos_gemv_bf16(yp, yn, wp, wn, xp, xn, m, k, _stream(stream)), "gemv_bf16")


def gemm_bf16(y, w, x, batch, m, k, stream=None):
    """gemm_bf16.rs:51-110: Y[batch, m] = X[batch, k] W[m, k]^T on MFMA."""
    yp, yn = _f32(y, "y")
    wp, wn = _w16(w, "w")
    xp, xn = _f32(x, "x")
    _check(lib().myos_gemm_bf16(yp, yn, wp, wn, xp, xn, batch, m, k, _stream(stream)),
           "gemm_bf16")


def gemm_bf16_noalloc(y, w, x, batch, m, k, stream=None):
    """gemm_bf16 with its scratch in the library's static device array (no
    allocation); Scratch error past myos_gemm_bf16_noalloc_max_scratch()."""
    yp, yn = _f32(y, "y")
    wp, wn = _w16(w, "w")
    xp, xn = _f32(x, "x")
    _check(lib().myos_gemm_bf16_noalloc(yp, yn, wp, wn, xp, xn, batch, m, k, _stream(stream)),
           "gemm_bf16_noalloc")


def add_bf16_bias(y, bias, stream=None):
    """bf16.rs:147-158."""
    yp, yn = _f32(y, "y")
    bp, bn = _w16(bias, "bias")
    _check(lib().myos_add_bf16_bias(yp, yn, bp, bn, _stream(stream)), "add_bf16_bias")


def embed_gather_bf16(out, table, shape, token_id, stream=None):
    """bf16.rs:165-198; shape = (vocab, hidden)."""
    if len(shape) != 2:
        raise MyosError(E_SHAPE, "embed_gather_bf16")
    op, on = _f32(out, "out")
    tp, tn = _w16(table, "table")
    _check(lib().myos_embed_gather_bf16(op, on, tp, tn, shape[0], shape[1], token_id,
                                        _stream(stream)), "embed_gather_bf16")


def rmsnorm_bf16_weight(y, weight, x, eps, stream=None):
    """bf16.rs:231-249."""
    yp, yn = _f32(y, "y")
    wp, wn = _w16(weight, "weight")
    xp, xn = _f32(x, "x")
    _check(lib().myos_rmsnorm_bf16_weight(yp, yn, wp, wn, xp, xn, eps, _stream(stream)),
           "rmsnorm_bf16_weight")


def rope_f32_inplace(x, position, head_dim, theta, stream=None):
    """rope.rs:119-126 (NeoX half-rotate)."""
    xp, xn = _f32(x, "x")
    _check(lib().myos_rope_f32_inplace(xp, xn, position, head_dim, theta, _stream(stream)),
           "rope_f32_inplace")


def gqa_attn_f32(y, q, k, v, probs, num_q_heads, num_kv_heads, head_dim, seq_len,
                 causal_pos=None, stream=None):
    """gqa.rs:174-218; causal_pos=None is GqaMask::Full, else Causal{query_pos}."""
    yp, yn = _f32(y, "y")
    qp, qn = _f32(q, "q")
    kp, kn = _f32(k, "k")
    vp, vn = _f32(v, "v")
    pp, pn = _f32(probs, "probs")
    mask = 0 if causal_pos is None else 1
    _check(lib().myos_gqa_attn_f32(yp, yn, qp, qn, kp, kn, vp, vn, pp, pn, num_q_heads,
                                   num_kv_heads, head_dim, seq_len, mask,
                                   0 if causal_pos is None else causal_pos, _stream(stream)),
           "gqa_attn_f32")


def swiglu_mul_f32(h, gate, up, stream=None):
    """swiglu.rs:125-131."""
    hp, hn = _f32(h, "h")
    gp, gn = _f32(gate, "gate")
    up_, un = _f32(up, "up")
    _check(lib().myos_swiglu_mul_f32(hp, hn, gp, gn, up_, un, _stream(stream)),
           "swiglu_mul_f32")


def swiglu_bf16(y, x, gate_w, up_w, down_w, gate, up, h, hidden, intermediate, stream=None):
    """swiglu.rs:184-213: y = W_d (silu(W_g x) * (W_u x)); gate/up/h scratch."""
    args = [_f32(y, "y"), _f32(x, "x"), _w16(gate_w, "gate_w"), _w16(up_w, "up_w"),
            _w16(down_w, "down_w"), _f32(gate, "gate"), _f32(up, "up"), _f32(h, "h")]
    flat = [v for pn in args for v in pn]
    _check(lib().myos_swiglu_bf16(*flat, hidden, intermediate, _stream(stream)), "swiglu_bf16")


def silu_f32(y, z, stream=None):
    """swiglu.rs:113-115, elementwise."""
    yp, yn = _f32(y, "y")
    zp, zn = _f32(z, "z")
    _check(lib().myos_silu_f32(yp, yn, zp, zn, _stream(stream)), "silu_f32")


def rmsnorm_f32(y, weight, x, eps, stream=None):
    """bf16.rs:200-216 (f32 gamma)."""
    yp, yn = _f32(y, "y")
    wp, wn = _f32(weight, "weight")
    xp, xn = _f32(x, "x")
    _check(lib().myos_rmsnorm_f32(yp, yn, wp, wn, xp, xn, eps, _stream(stream)), "rmsnorm_f32")


def rope_inv_freqs(inv_freq, head_dim, theta, stream=None):
    """rope.rs:89-98 into a device tensor of head_dim / 2 floats."""
    ip, n = _f32(inv_freq, "inv_freq")
    _check(lib().myos_rope_inv_freqs(ip, n, head_dim, theta, _stream(stream)), "rope_inv_freqs")


def attn_scale_f32(head_dim) -> float:
    """gqa.rs:158-163."""
    out = C.c_float()
    _check(lib().myos_attn_scale_f32(head_dim, C.byref(out)), "attn_scale_f32")
    return out.value


def greedy_token(logits, out=None, stream=None) -> int:
    """model_core/src/lib.rs:157-167; returns the id (syncs the stream)."""
    import torch
    if out is None:
        out = torch.zeros(1, dtype=torch.int32, device=logits.device)
    lp, ln = _f32(logits, "logits")
    op, _ = _dev(out, "out")
    s = _stream(stream)
    _check(lib().myos_greedy_token(op, lp, ln, s), "greedy_token")
    _check(lib().myos_stream_sync(s), "greedy_token sync")
    return int(out.view(torch.int32).cpu()[0].item()) & 0xFFFFFFFF


# ------------------------------------------------------------- model tier ----

class Model:
    """model_core over one GPU: weights in HBM, KvCache [layers][kv][max_seq][d]."""

    def __init__(self, handle, shape: BlockShape):
        self._h = handle
        self.shape = shape

    @classmethod
    def open(cls, path: str, shape: BlockShape | None = None, kv_dtype: int = KV_F32,
             max_seq: int = 256) -> "Model":
        shape = shape or preset(SHAPE_QWEN25_1_5B)
        h = C.c_void_p()
        _check(lib().myos_model_open(os.fsencode(path), C.byref(shape), kv_dtype, max_seq,
                                     C.byref(h)), f"open {path}")
        return cls(h, shape)

    def close(self):
        if getattr(self, "_h", None):
            lib().myos_model_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def prefill(self, tokens):
        import numpy as np
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        _check(lib().myos_prefill(self._h, t.ctypes.data_as(P), t.size), "prefill")

    def forward_token(self, token: int, pos: int):
        _check(lib().myos_forward_token(self._h, token, pos), "forward_token")

    def greedy_decode(self, steps: int):
        import numpy as np
        out = np.zeros(max(steps, 1), np.uint32)
        before = self.cache_len()
        rc = lib().myos_greedy_decode(self._h, steps, out.ctypes.data_as(P))
        if rc != OK:
            # like the reference's loop, ids of the steps that ran are kept
            err = MyosError(rc, "greedy_decode")
            err.partial = [int(v) for v in out[:self.cache_len() - before]]
            raise err
        return [int(v) for v in out[:steps]]

    def decode_forced(self, ids):
        """Teacher-forced steps: step s feeds ids[s]; returns the greedy
        argmax of the logits each step started from."""
        import numpy as np
        t = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(max(t.size, 1), np.uint32)
        _check(lib().myos_decode_forced(self._h, t.ctypes.data_as(P), t.size,
                                        out.ctypes.data_as(P)), "decode_forced")
        return [int(v) for v in out[:t.size]]

    def attention_layer(self, layer: int, pos: int, residual, proj_in):
        """attn_wire.rs:207-313 on the model's weights: returns residual +
        o_proj(attention(proj_in)); stores the layer's K/V row at pos (the
        cursor does not move: kv_advance)."""
        import numpy as np
        r = np.array(residual, dtype=np.float32, copy=True)
        x = np.ascontiguousarray(proj_in, dtype=np.float32)
        if r.size != x.size:
            raise MyosError(E_SHAPE, "attention_layer")
        _check(lib().myos_attention_layer(self._h, layer, pos, r.ctypes.data_as(P),
                                          x.ctypes.data_as(P), r.size), "attention_layer")
        return r

    def kv_advance(self):
        """KvCache::advance (kv_cache.rs:226-232)."""
        _check(lib().myos_kv_advance(self._h), "kv_advance")

    def debug_raise_wait_error(self):
        """Test hook: the next persistent launch's waits give up at once."""
        _check(lib().myos_debug_raise_wait_error(self._h), "debug_raise_wait_error")

    def cache_len(self) -> int:
        return int(lib().myos_cache_len(self._h))

    def cache_clear(self):
        """KvCache::clear (kv_cache.rs:234-237): cursor to 0, slots kept."""
        _check(lib().myos_cache_clear(self._h), "cache_clear")

    def time_kernel(self, which: int, reps: int = 20) -> float:
        """Average ms of one decode kernel launch (clobbers activations)."""
        out = C.c_double()
        _check(lib().myos_time_kernel(self._h, which, reps, C.byref(out)), "time_kernel")
        return out.value

    def kernel_bytes(self, which: int) -> float:
        return float(lib().myos_kernel_bytes(self._h, which))

    def max_seq(self) -> int:
        return int(lib().myos_max_seq(self._h))

    def _copy(self, fn, n):
        import numpy as np
        out = np.zeros(n, np.float32)
        _check(fn(self._h, out.ctypes.data_as(P), n), fn.__name__)
        return out

    def logits(self):
        return self._copy(lib().myos_copy_logits, self.shape.vocab)

    def hidden(self):
        return self._copy(lib().myos_copy_hidden, self.shape.hidden)

    def normed(self):
        return self._copy(lib().myos_copy_normed, self.shape.hidden)

    def kv(self, layer, head, pos):
        import numpy as np
        d = self.shape.head_dim
        k = np.zeros(d, np.float32)
        v = np.zeros(d, np.float32)
        _check(lib().myos_kv_read(self._h, layer, head, pos, k.ctypes.data_as(P),
                                  v.ctypes.data_as(P)), "kv_read")
        return k, v

    def set_graph(self, on: bool):
        _check(lib().myos_set_graph(self._h, 1 if on else 0), "set_graph")

    def set_decode_mode(self, mode: int):
        """DECODE_AUTO / DECODE_KERNELS / DECODE_PERSISTENT / DECODE_STREAMED for
        greedy_decode."""
        _check(lib().myos_set_decode_mode(self._h, int(mode)), "set_decode_mode")

    def set_decode_trace(self, step: int):
        """Record phase timestamps of decode step `step` of each persistent
        greedy_decode call (step < 0: off)."""
        _check(lib().myos_set_decode_trace(self._h, int(step)), "set_decode_trace")

    def decode_trace(self):
        """[256 workgroups, 5 * layers + 3] device clock ticks (100 MHz)."""
        import numpy as np
        out = np.zeros((256, 5 * self.shape.num_layers + 3), np.uint64)
        _check(lib().myos_copy_decode_trace(self._h, out.ctypes.data_as(P), out.size),
               "copy_decode_trace")
        return out

    def decode_path(self) -> int:
        """DECODE_KERNELS, DECODE_PERSISTENT or DECODE_STREAMED: the path
        greedy_decode takes."""
        return int(lib().myos_decode_path(self._h))

    def last_prefill_ms(self) -> float:
        return float(lib().myos_last_prefill_ms(self._h))

    def last_decode_ms(self) -> float:
        return float(lib().myos_last_decode_ms(self._h))

    def weight_bytes(self) -> int:
        return int(lib().myos_weight_bytes(self._h))

    def kv_bytes(self) -> int:
        return int(lib().myos_kv_bytes(self._h))


def sha256_file(path: str) -> str:
    """SHA-256 of a file (hex), the run fingerprint's model_sha256."""
    out = C.create_string_buffer(65)
    _check(lib().myos_sha256_file(os.fsencode(path), out), f"sha256 {path}")
    return out.value.decode()


def write_random_qwen25(path: str, shape: BlockShape | None = None, seed: int = 0,
                        std: float = 0.02, threads: int | None = None):
    """Seeded N(0, std) BF16 weights in qwen25_layout keys (norm gains 1.0)."""
    shape = shape or preset(SHAPE_QWEN25_1_5B)
    threads = threads or min(16, os.cpu_count() or 1)
    _check(lib().myos_write_random_qwen25(os.fsencode(path), C.byref(shape), seed, std, threads),
           f"write {path}")
