"""Pins the CPU oracle against the reference's own known answers.

Every expected value below is a constant the reference's tests hard-code
(file:line cited), or a closed form / brute-force bound that a plausible
mistake (dropped term, wrong sign or index, reordered sum) would break.
"""
import math

import numpy as np
import pytest

from model_fixtures import bits, block_fixture, fixture_shape, rich_map, rich_shape, THETA


def fb(x):
    return int(np.float32(x).view(np.uint32))


def fbits(a):
    return [int(v) for v in np.asarray(a, np.float32).view(np.uint32)]


# ------------------------------------------------------------ bf16.rs ----

def test_eps_bits():
    # bf16.rs:311
    assert fb(np.float32(1e-6)) == 0x358637BD


def test_bf16_decode(orc):
    # bf16.rs:316-320 (LE byte pairs -> u16)
    assert orc.lib().orc_bf16_to_f32(0x3F80) == 1.0
    assert orc.lib().orc_bf16_to_f32(0xC000) == -2.0
    assert fb(orc.lib().orc_bf16_to_f32(0x803F)) == 0x803F0000


def test_add_bias_hand_values(orc):
    # bf16.rs:324-333
    y = orc.add_bf16_bias([10.0, 20.0], bits([0.5, 1.0]))
    assert list(y) == [10.5, 21.0]


def test_gemv_hand_values(orc):
    # bf16.rs:350-362: W=[[1,2,.5],[-1,4,1.5]], x=[1,-2,.5] -> [-2.75,-8.25]
    w = bits([1.0, 2.0, 0.5, -1.0, 4.0, 1.5])
    x = [1.0, -2.0, 0.5]
    assert list(orc.gemv_bf16(w, x, 2, 3)) == [-2.75, -8.25]
    assert list(orc.gemv_bf16(w, x, 2, 3, threads=3)) == [-2.75, -8.25]


def test_gemv_le_weights(orc):
    # bf16.rs:379-387
    assert orc.gemv_bf16(np.array([0x3F80], np.uint16), [2.0], 1, 1)[0] == 2.0
    y = orc.gemv_bf16(np.array([0x803F], np.uint16), [2.0], 1, 1)[0]
    assert y == np.float32(np.uint32(0x803F0000).view(np.float32)) * np.float32(2.0)


def test_gemv_zero_k(orc):
    # bf16.rs:366-371: k == 0 fills zero
    y = orc.gemv_bf16(np.zeros(0, np.uint16), np.zeros(0, np.float32), 2, 0)
    assert list(y) == [0.0, 0.0]


@pytest.mark.parametrize("rows", [1, 8, 32, 40])
def test_gemv_order_cancellation(orc, rows):
    # gemv_bf16_kernel.rs:929-951: [2^24,1,1,1,-2^24,1,1,1] . ones -> 3 (not 0 or 4),
    # for single rows and inside 8/32-row panels.
    row = [16777216.0, 1.0, 1.0, 1.0, -16777216.0, 1.0, 1.0, 1.0]
    w = bits(np.tile(row, rows))
    for threads in (0, 1, 3, 8):
        y = orc.gemv_bf16(w, np.ones(8, np.float32), rows, 8, threads=threads)
        assert np.all(y == 3.0)


def _gemv_scalar_ref(w_bits, x):
    # direct f32 chain in numpy (one rounding per op) -- slow, tiny shapes only
    wf = (w_bits.astype(np.uint32) << 16).view(np.float32)
    out = np.zeros(wf.shape[0], np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        _chain(wf, x, out)
    return out


def _chain(wf, x, out):
    for i in range(wf.shape[0]):
        acc = np.float32(0)
        for j in range(wf.shape[1]):
            acc = np.float32(acc + np.float32(wf[i, j] * x[j]))
        out[i] = acc


@pytest.mark.parametrize("m,k", [(1, 1), (7, 3), (9, 17), (33, 24), (40, 31)])
def test_gemv_scalar_avx_threads_bit_equal(orc, m, k):
    # gemv_bf16_kernel.rs:878-899,969-1029,1282-1323: every path and thread count
    # is bit-equal to the left-to-right chain, including row and column tails.
    rng = np.random.default_rng(m * 100 + k)
    w = rng.integers(0, 65536, size=(m, k), dtype=np.uint16)
    w[(w & 0x7F80) == 0x7F80] = 0x3F80  # keep NaN/inf out of this sweep
    x = rng.standard_normal(k).astype(np.float32)
    ref = _gemv_scalar_ref(w, x)
    assert fbits(orc.gemv_bf16(w, x, m, k)) == fbits(ref)
    for t in (1, 2, 3, 7, 8):
        assert fbits(orc.gemv_bf16(w, x, m, k, threads=t)) == fbits(ref)


def test_gemv_all_bf16_patterns(orc):
    # gemv_bf16_kernel.rs:1032-1048: all 65536 bf16 patterns as one column,
    # x = 1 -> y is exactly the decoded weight (NaN payloads preserved).
    w = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(65536, 1)
    y = orc.gemv_bf16(w, np.ones(1, np.float32), 65536, 1, threads=4)
    expect = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    nan = np.isnan(expect)
    assert np.all(np.isnan(y[nan]))
    assert fbits(y[~nan]) == fbits(expect[~nan] * np.float32(1.0) + np.float32(0.0))


def test_gemv_forward_error_bound(orc):
    # brute force in float64: |y - exact| <= gamma_k * sum|w||x| (Higham 3.1)
    rng = np.random.default_rng(5)
    m, k = 64, 1536
    w = (rng.standard_normal((m, k)).astype(np.float32) * 0.02)
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)
    wf = (wb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x = rng.standard_normal(k).astype(np.float32)
    y = orc.gemv_bf16(wb, x, m, k, threads=4).astype(np.float64)
    exact = wf @ x.astype(np.float64)
    u = 2.0 ** -24
    bound = (k * u / (1 - k * u)) * (np.abs(wf) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - exact) <= bound)


def test_gemm_equals_per_token_gemv(orc):
    # gemm_bf16.rs:517-572: Y[b] is bit-identical to gemv(X[b])
    rng = np.random.default_rng(9)
    m, k, b = 70, 45, 5
    w = (rng.standard_normal((m, k)).astype(np.float32) * 0.02).view(np.uint32) >> 16
    w = w.astype(np.uint16)
    x = rng.standard_normal((b, k)).astype(np.float32)
    y = orc.gemm_bf16(w, x, b, m, k, threads=3)
    for i in range(b):
        assert fbits(y[i]) == fbits(orc.gemv_bf16(w, x[i], m, k))


def test_embed_gather(orc):
    # bf16.rs:381-396
    table = bits([1.0, 2.0, 3.0, -0.5, 0.5, 4.0])
    assert list(orc.embed_gather_bf16(table, 3, 2, 1)[1]) == [3.0, -0.5]
    assert list(orc.embed_gather_bf16(table, 3, 2, 2)[1]) == [0.5, 4.0]
    assert list(orc.embed_gather_bf16(table, 3, 2, 0)[1]) == [1.0, 2.0]
    rc, _ = orc.embed_gather_bf16(table, 3, 2, 3)
    assert rc == 2  # TokenOutOfBounds


def test_rmsnorm_hand_values(orc):
    # bf16.rs:469-486
    y = orc.rmsnorm_bf16_weight(bits([1.5, 4.0, -2.0, 0.5]), [8.0, 0, 0, 0], 0.0)
    assert list(y) == [3.0, 0.0, 0.0, 0.0]
    y = orc.rmsnorm_bf16_weight(bits([3.0, 4.0]), [2.0, -2.0], 0.0)
    assert list(y) == [3.0, -4.0]


def test_rmsnorm_serial_order(orc):
    # bf16.rs:488-506: Sum x^2 left to right keeps 2^24 -> y = [2, 2^-11 x3]
    y = orc.rmsnorm_bf16_weight(bits([1.0] * 4), [4096.0, 1.0, 1.0, 1.0], 0.0)
    assert fbits(y) == [fb(2.0)] + [0x3A000000] * 3


def test_rmsnorm_eps_bits(orc):
    # bf16.rs:508-531: 1/sqrt(1 + 1e-6) -> 0x3f7ffff8; zeros stay zero with eps
    y = orc.rmsnorm_bf16_weight(bits([1.0] * 4), [1.0] * 4, np.float32(1e-6))
    assert fbits(y) == [0x3F7FFFF8] * 4
    y = orc.rmsnorm_bf16_weight(bits([3.0, -1.0]), [0.0, 0.0], np.float32(1e-6))
    assert list(y) == [0.0, 0.0]
    y = orc.rmsnorm_bf16_weight(bits([3.0, -1.0]), [0.0, 0.0], 0.0)
    assert np.all(np.isnan(y))


# ------------------------------------------------------------- rope.rs ---

def test_rope_theta_bits():
    assert fb(THETA) == 0x49742400  # rope.rs:230


def test_rope_identity_at_zero(orc):
    # rope.rs:237-258
    x = np.array([1.0, -2.0, 3.5, -4.25], np.float32)
    assert list(orc.rope_f32_inplace(x, 0, 4, THETA)[1]) == list(x)
    wide = np.array([(i + 0.5) if i % 2 == 0 else -(i + 0.25) for i in range(128)], np.float32)
    assert fbits(orc.rope_f32_inplace(wide, 0, 128, THETA)[1]) == fbits(wide)


def test_rope_one_radian(orc):
    # rope.rs:262-280
    assert fbits(orc.rope_f32_inplace([1.0, 0.0], 1, 2, THETA)[1]) == [0x3F0A5140, 0x3F576AA4]
    assert fbits(orc.rope_f32_inplace([3.0, 4.0], 1, 2, THETA)[1]) == [0xBFDF5B68, 0x4095F09E]


def test_rope_second_pair_table(orc):
    # rope.rs:283-307
    t = orc.rope_inv_freqs(4, THETA)
    assert fbits(t) == [fb(1.0), 0x3A83126F]
    y = orc.rope_f32_inplace([0.0, 1.0, 0.0, 0.0], 1, 4, THETA)[1]
    assert fbits(y) == [0, 0x3F7FFFF8, 0, 0x3A83126E]


def test_rope_position_three(orc):
    # rope.rs:310-325
    y = orc.rope_f32_inplace([1.0, 2.0, 3.0, 4.0], 3, 4, THETA)[1]
    assert fbits(y) == [0xBFB4E8BC, 0x3FFE767E, 0xC0350C00, 0x40803101]
    both = orc.rope_f32_inplace([1.0, 2.0, 3.0, 4.0] * 2, 3, 4, THETA)[1]
    assert fbits(both[:4]) == fbits(y) and fbits(both[4:]) == fbits(y)


def test_rope_qwen_head_neox(orc):
    # rope.rs:328-361
    x = np.zeros(128, np.float32)
    x[0] = 1.0
    y = orc.rope_f32_inplace(x, 1, 128, THETA)[1]
    assert fb(y[0]) == 0x3F0A5140 and fb(y[64]) == 0x3F576AA4 and y[1] == 0 and y[127] == 0
    t = orc.rope_inv_freqs(128, THETA)
    assert fb(t[0]) == fb(1.0) and fb(t[32]) == fb(np.float32(1.0) / np.float32(1000.0))
    assert fb(t[63]) == 0x35A68E4C
    last = np.zeros(128, np.float32)
    last[63], last[127] = 1.0, -2.0
    y = orc.rope_f32_inplace(last, 8, 128, THETA)[1]
    assert fb(y[63]) == 0x3F8000A7 and fb(y[127]) == 0xBFFFFFAD and y[62] == 0 and y[1] == 0


def test_rope_rejects_bad_shapes(orc):
    # rope.rs:364-430 (Shape errors)
    assert orc.rope_f32_inplace([1.0, 2.0, 3.0, 4.0, 5.0], 1, 4, THETA)[0] == 1
    assert orc.rope_f32_inplace([9.0, 8.0, 7.0], 1, 3, THETA)[0] == 1
    assert orc.rope_f32_inplace([1.0, 2.0], 0, 0, THETA)[0] == 1


# -------------------------------------------------------------- gqa.rs ---

def test_gqa_scale_bits(orc):
    # gqa.rs:357-363
    assert fb(orc.attn_scale_f32(1)) == 0x3F800000
    assert fb(orc.attn_scale_f32(4)) == 0x3F000000
    assert fb(orc.attn_scale_f32(128)) == 0x3DB504F3


def test_gqa_groups(orc):
    # gqa.rs:366-401: contiguous head groups, bits of the mix and last-head probs
    y, probs = orc.gqa_attn_f32([1, 1, 4, 4], [1, 0, 0, 2], [10, 0, 0, 7], 4, 2, 1, 2)
    assert fbits(y) == [0x40E9F052, 0x40E9F052, 0x40DFECC5, 0x40DFECC5]
    assert fbits(probs) == [0x39AFD1EF, 0x3F7FEA06]


def test_gqa_causal(orc):
    # gqa.rs:403-488
    q, k, v = [1, 1, 4, 4], [1, 0, 0, 2], [10, 0, 0, 7]
    y, probs = orc.gqa_attn_f32(q, k, v, 4, 2, 1, 2, causal_pos=0)
    assert list(y) == [10, 10, 0, 0] and list(probs) == [1, 0]
    yf, _ = orc.gqa_attn_f32(q, k, v, 4, 2, 1, 2)
    assert fbits(orc.gqa_attn_f32(q, k, v, 4, 2, 1, 2, causal_pos=1)[0]) == fbits(yf)
    assert fbits(orc.gqa_attn_f32(q, k, v, 4, 2, 1, 2, causal_pos=2 ** 63)[0]) == fbits(yf)
    y1, p1 = orc.gqa_attn_f32([50.0], [50.0], [3.5], 1, 1, 1, 1)
    assert list(y1) == [3.5] and list(p1) == [1.0]


def test_gqa_softmax_bits(orc):
    # gqa.rs:491-572
    q = [2.0, 0, 0, 0]
    k = np.zeros(8, np.float32)
    k[0] = 1
    v = np.zeros(8, np.float32)
    v[0], v[4] = 4, 8
    y, probs = orc.gqa_attn_f32(q, k, v, 1, 1, 4, 2)
    assert fbits(probs) == [0x3F3B26A8, 0x3E89B2B1]
    assert fb(y[0]) == 0x40A26CAC and list(y[1:]) == [0, 0, 0]
    yb, pb = orc.gqa_attn_f32([1.0], [100.0, 100.0], [2.0, 6.0], 1, 1, 1, 2)
    assert list(pb) == [0.5, 0.5] and list(yb) == [4.0]
    q = np.zeros(128, np.float32)
    q[0] = 1
    k = np.zeros(256, np.float32)
    k[0] = 1
    v = np.zeros(256, np.float32)
    v[0], v[128] = 2, 6
    y, probs = orc.gqa_attn_f32(q, k, v, 1, 1, 128, 2)
    assert fbits(probs) == [0x3F05A737, 0x3EF4B194]
    assert fb(y[0]) == 0x407A58CA and np.all(y[1:] == 0)


def test_gqa_dot_order(orc):
    # gqa.rs:575-609
    k = [16777216.0, 1, 1, 1, 1, 1, 1, 16777216.0]
    v = [2.0, 0, 0, 0, 8.0, 0, 0, 0]
    y, _ = orc.gqa_attn_f32([1.0] * 4, k, v, 1, 1, 4, 2)
    assert fb(y[0]) == 0x40E91CEF


def test_gqa_qwen_width_uniform(orc):
    # gqa.rs:611-650: Q = 0 -> uniform softmax; heads 0..5 read KV0, 6..11 KV1
    H = 128
    k = np.zeros(2 * 2 * H, np.float32)
    v = np.zeros(2 * 2 * H, np.float32)
    v[0], v[H] = 2.0, 6.0            # KV0, t0/t1 lane 0 -> mean 4
    v[2 * H], v[3 * H] = 10.0, 30.0  # KV1 -> mean 20
    y, _ = orc.gqa_attn_f32(np.zeros(12 * H), k, v, 12, 2, H, 2)
    y = y.reshape(12, H)
    assert np.all(y[:6, 0] == 4.0) and np.all(y[6:, 0] == 20.0)


# ----------------------------------------------------------- swiglu.rs ---

def test_silu_bits(orc):
    # swiglu.rs:362-377
    assert fb(orc.silu_f32(0.0)) == 0
    assert fb(orc.silu_f32(-0.0)) == 0x80000000
    assert fb(orc.silu_f32(1.0)) == 0x3F3B26A8
    assert fb(orc.silu_f32(-1.0)) == 0xBE89B2B1
    assert fb(orc.silu_f32(2.0)) == 0x3FE17BEA
    assert fb(orc.silu_f32(3.0)) == 0x4036E4ED
    assert fb(orc.silu_f32(-1.5)) == 0xBE8C1A51


def test_swiglu_mul_bits(orc):
    # swiglu.rs:379-388
    h = orc.swiglu_mul_f32([0.0, 1.0, -1.0, 3.0], [4.0, 2.0, -3.0, 0.5])
    assert fbits(h) == [0x00000000, 0x3FBB26A8, 0x3F4E8C0A, 0x3FB6E4ED]


def test_swiglu_mlp_bits(orc):
    # swiglu.rs:392-452: gate/up/down composition through the GEMV
    x = [1.0, 0.0]
    g = orc.gemv_bf16(bits([1.0, 0.0, 0.0, 1.0]), x, 2, 2)
    u = orc.gemv_bf16(bits([2.0, 3.0, 0.0, 5.0]), x, 2, 2)
    h = orc.swiglu_mul_f32(g, u)
    y = orc.gemv_bf16(bits([0.5, 3.0, 1.0, 5.0]), h, 2, 2)
    assert fbits(h) == [0x3FBB26A8, 0] and fbits(y) == [0x3F3B26A8, 0x3FBB26A8]


# ------------------------------------------------------------- argmax ----

def test_greedy_token_spec(orc):
    # model_core/src/lib.rs:157-167: strict >, lowest index on ties, NaN never wins
    assert orc.greedy_token([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.greedy_token([np.nan, 1.0, np.nan]) == 1
    assert orc.greedy_token([np.nan, np.nan]) == 0
    assert orc.greedy_token([-np.inf, -np.inf]) == 0
    assert orc.greedy_token([-np.inf, -1e30]) == 1
    assert orc.greedy_token([np.inf, np.inf, 5.0]) == 0


# -------------------------------------------------------- model tier ----

def test_block_fixture_forward(orc):
    # qwen25_block.rs:1011-1071: token 0 -> logits [1, 2, 0, -1], KV slot values
    s, t = block_fixture()
    m = orc.Model(s, t, 4, threads=1)
    assert m.forward_token(0, 0) == 0
    assert list(m.logits()) == [1.0, 2.0, 0.0, -1.0]
    assert m.cache_len() == 1
    k, v = m.kv(0, 0, 0)
    assert list(k) == [0.0, 0.0] and list(v) == [1.0, 0.0]
    k, v = m.kv(0, 0, 1)
    assert list(k) == [0.0, 0.0] and list(v) == [0.0, 0.0]


def test_block_fixture_prefill_decode(orc):
    # qwen25_block.rs:1200-1221: prefill [0] then 4 greedy steps -> [1, 1, 1, 1]
    s, t = block_fixture()
    m = orc.Model(s, t, 8, threads=2)
    assert m.prefill([]) == 1
    assert m.cache_len() == 0
    assert m.prefill([0]) == 0
    assert list(m.logits()) == [1.0, 2.0, 0.0, -1.0]
    rc, out = m.greedy_decode(4)
    assert rc == 0 and list(out) == [1, 1, 1, 1] and m.cache_len() == 5
    assert list(m.kv(0, 0, 4)[1]) == [1.0, 0.0]


def test_block_errors_do_not_advance(orc):
    # qwen25_block.rs:1224-1300
    s, t = block_fixture()
    m = orc.Model(s, t, 2, threads=1)
    assert m.forward_token(0, 1) == 4   # Position
    assert m.forward_token(9, 0) == 2   # Token
    assert m.cache_len() == 0
    full = orc.Model(s, t, 1, threads=1)
    assert full.forward_token(0, 0) == 0
    before = full.logits()
    assert full.forward_token(1, 1) == 5  # KV full
    assert full.cache_len() == 1 and list(full.logits()) == list(before)
    assert m.prefill([0, 9]) == 2 and m.cache_len() == 0
    small = orc.Model(s, t, 2, threads=1)
    assert small.prefill([0, 0, 0]) == 5 and small.cache_len() == 0


def _rms_f32(x, gamma, eps):
    """RMSNorm in the reference's f32 order (bf16.rs:243-270): serial sum of
    squares, mean, 1/sqrt(mean + eps), g * (x * inv)."""
    x = np.asarray(x, np.float32)
    s = np.float32(0)
    for v in x:
        s = np.float32(s + np.float32(v * v))
    inv = np.float32(1) / np.float32(math.sqrt(np.float32(s / np.float32(len(x)) + eps)))
    return np.asarray([np.float32(g * np.float32(v * inv)) for g, v in zip(gamma, x)],
                      np.float32)


def _fixture_head(normed):
    """Tied head of the fixture embedding rows [1,1], [2,0], [0,4], [-1,0]."""
    n0, n1 = np.float32(normed[0]), np.float32(normed[1])
    rows = [(1, 1), (2, 0), (0, 4), (-1, 0)]
    return [np.float32(np.float32(np.float32(a) * n0) + np.float32(np.float32(b) * n1))
            for a, b in rows]


def test_swiglu_residual_changes_the_logits(orc):
    # qwen25_block.rs:1074-1129: the stream is [2, 2] before the MLP, its
    # post-norm [1, 1]; gate and up read lane 0, so h = [silu(1) * 1, 0] and
    # down (identity) adds [silu(1), 0]. silu(1) = 0x3F3B26A8 (swiglu.rs:362-377).
    from model_fixtures import swiglu_residual_fixture
    s, t = swiglu_residual_fixture()
    silu1 = np.uint32(0x3F3B26A8).view(np.float32)
    residual = [np.float32(2.0 + silu1), np.float32(2.0)]
    expect = _fixture_head(_rms_f32(residual, [1.0, 0.0], np.float32(0)))
    assert expect != [1.0, 2.0, 0.0, -1.0]
    m = orc.Model(s, t, 2, threads=1)
    assert m.forward_token(0, 0) == 0
    assert fbits(m.logits()) == fbits(expect)
    assert fbits(m.hidden()) == fbits(residual)
    assert m.cache_len() == 1
    assert list(m.kv(0, 0, 0)[1]) == [1.0, 0.0]
    # the prefill chunk path gives the same bits
    mp = orc.Model(s, t, 2, threads=1)
    assert mp.prefill([0]) == 0 and fbits(mp.logits()) == fbits(expect)


def test_two_layers_advance_once_per_token(orc):
    # qwen25_block.rs:1132-1197
    from model_fixtures import two_layer_fixture
    s, t = two_layer_fixture()
    for use_prefill in (False, True):
        m = orc.Model(s, t, 4, threads=1)
        if use_prefill:
            assert m.prefill([0]) == 0
        else:
            assert m.forward_token(0, 0) == 0
        assert list(m.logits()) == [1.0, 2.0, 0.0, -1.0]
        assert m.cache_len() == 1
        assert list(m.kv(0, 0, 0)[1]) == [2.0, 0.0] and list(m.kv(1, 0, 0)[1]) == [0.0, 8.0]
        assert list(m.kv(0, 0, 0)[0]) == [0.0, 0.0] and list(m.kv(1, 0, 0)[0]) == [0.0, 0.0]
        assert list(m.kv(0, 0, 1)[1]) == [0.0, 0.0] and list(m.kv(1, 0, 1)[1]) == [0.0, 0.0]
        assert m.forward_token(1, 1) == 0
        assert m.cache_len() == 2
        assert list(m.kv(0, 0, 0)[1]) == [2.0, 0.0] and list(m.kv(1, 0, 0)[1]) == [0.0, 8.0]
        assert list(m.kv(0, 0, 1)[1]) == [2.0, 0.0] and list(m.kv(1, 0, 1)[1]) == [0.0, 8.0]
        # token 1 embeds to [2, 0]; attention and SwiGLU add 0; final gamma [1, 0]
        expect = _fixture_head(_rms_f32([2.0, 0.0], [1.0, 0.0], np.float32(0)))
        assert fbits(m.logits()) == fbits(expect)
        assert expect[1] > expect[0] and orc.greedy_token(m.logits()) == 1


def test_post_attention_norm_feeds_the_mlp(orc):
    # Closed form on the fixture shape, chosen so that the plausible wiring
    # mistakes give different logits: ln2 gamma [2, 0] (ln1 stays [1, 1]), so
    # the MLP input is rms([2, 2]) * [2, 0] = [2, 0], not the ln1-normed [1, 1];
    # gate = [[1,0],[0,0]], up = identity: h = [silu(2) * 2, 0] with
    # silu(2) = 0x3FE17BEA (swiglu.rs:362-377); down = [[1,0],[0.5,0]] adds
    # [h0, h0 / 2] to the stream; final gamma [1, 0.5].
    from model_fixtures import block_fixture_layer, fixture_embed_and_final
    s = fixture_shape()
    t = fixture_embed_and_final((1.0, 0.5))
    block_fixture_layer(t, 0, [0.0] * 4, [1.0, 0.0], [1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0],
                        [1.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 1.0], [1.0, 0.0, 0.5, 0.0])
    t["model.layers.0.post_attention_layernorm.weight"] = bits([2.0, 0.0])
    silu2 = np.uint32(0x3FE17BEA).view(np.float32)
    n2 = _rms_f32([2.0, 2.0], [2.0, 0.0], np.float32(0))
    assert list(n2) == [2.0, 0.0]
    h0 = np.float32(silu2 * np.float32(2.0))
    x = [np.float32(2.0 + h0), np.float32(2.0 + np.float32(0.5 * h0))]
    expect = _fixture_head(_rms_f32(x, [1.0, 0.5], np.float32(0)))
    m = orc.Model(s, t, 2, threads=1)
    assert m.forward_token(0, 0) == 0
    assert fbits(m.hidden()) == fbits(x)
    assert fbits(m.logits()) == fbits(expect)
    # the wrong wirings: MLP on the ln1-normed [1, 1], or no MLP residual
    silu1 = np.uint32(0x3F3B26A8).view(np.float32)
    wrong = [_fixture_head(_rms_f32([2.0 + silu1, 2.0 + 0.5 * silu1], [1.0, 0.5], 0.0)),
             _fixture_head(_rms_f32([2.0, 2.0], [1.0, 0.5], 0.0))]
    assert all(fbits(w) != fbits(expect) for w in wrong)


def test_untied_head_copy_equals_tied(orc):
    # An lm_head.weight equal to the embedding gives bit-identical logits to
    # the tied head (the 7B checkpoint's untied head is the same GEMV over a
    # different matrix); a different lm_head moves them.
    from model_fixtures import random_map, shape_dict
    s = shape_dict(64, 4, 2, 16, 96, 50, 2, 1e-6)
    t = random_map(s, seed=3, std=0.1)
    tied = orc.Model(s, t, 8, threads=1)
    tu = dict(t)
    tu["lm_head.weight"] = np.array(t["model.embed_tokens.weight"], copy=True)
    untied = orc.Model(s, tu, 8, threads=1)
    td = dict(t)
    td["lm_head.weight"] = random_map(s, seed=4, std=0.1)["model.embed_tokens.weight"]
    other = orc.Model(s, td, 8, threads=1)
    for m in (tied, untied, other):
        assert m.prefill([5, 7, 9]) == 0
        assert m.forward_token(11, 3) == 0
    assert fbits(untied.logits()) == fbits(tied.logits())
    assert fbits(other.hidden()) == fbits(tied.hidden())
    assert fbits(other.logits()) != fbits(tied.logits())
    from qwen2_textbook import Textbook
    tb = Textbook(s, td)
    for tok in (5, 7, 9, 11):
        lg, _, _ = tb.forward(tok)
    assert np.max(np.abs(other.logits() - lg)) / np.max(np.abs(lg)) < 1e-5


@pytest.mark.parametrize("dims,seed", [((32, 4, 2, 8, 48, 40, 3), 1),
                                       ((48, 6, 1, 8, 64, 33, 2), 2),
                                       ((64, 4, 4, 16, 80, 50, 4), 3)])
def test_oracle_matches_textbook_forward(orc, dims, seed):
    # The oracle's f32 composition against the independent f64 forward on
    # random models with random (not unit) norm gains, so ln1 / ln2 / final
    # mix-ups, a dropped residual or a wrong layer's cache would all show.
    from model_fixtures import random_map, rne_bf16, shape_dict
    from qwen2_textbook import Textbook
    s = shape_dict(*dims, 1e-6)
    t = random_map(s, seed=seed, std=0.2)
    rng = np.random.default_rng(seed + 100)
    for name in t:
        if name.endswith("norm.weight"):
            t[name] = rne_bf16(rng.uniform(0.5, 1.5, t[name].shape).astype(np.float32))
    tb = Textbook(s, t)
    m = orc.Model(s, t, 16, threads=2)
    prompt = [int(v) for v in rng.integers(0, s["vocab"], 5)]
    assert m.prefill(prompt) == 0
    for tok in prompt:
        lg, hid, nrm = tb.forward(tok)
    rel = lambda a, b: float(np.max(np.abs(a - b)) / np.max(np.abs(b)))
    assert rel(m.logits(), lg) < 1e-5 and rel(m.hidden(), hid) < 1e-5
    assert rel(m.normed(), nrm) < 1e-5
    for step in range(6):
        tok = int(np.argmax(lg))
        assert m.forward_token(tok, m.cache_len()) == 0
        lg, hid, _ = tb.forward(tok)
        assert rel(m.logits(), lg) < 1e-5, step
        assert rel(m.hidden(), hid) < 1e-5, step
    for l in range(s["num_layers"]):
        for h in range(s["num_kv_heads"]):
            for p in (0, 4, 10):
                k, v = m.kv(l, h, p)
                kt, vt = tb.kv(l, h, p)
                assert rel(k, kt) < 1e-5 and rel(v, vt) < 1e-5, (l, h, p)


def _serial(m, tokens, start):
    last = None
    for i, tok in enumerate(tokens):
        assert m.forward_token(tok, start + i) == 0
        last = m.logits()
    return last


def _kv_bits(m, s, length):
    out = []
    for l in range(s["num_layers"]):
        for h in range(s["num_kv_heads"]):
            for p in range(length):
                k, v = m.kv(l, h, p)
                out += fbits(k) + fbits(v)
    return out


def test_chunk_prefill_equals_serial(orc):
    # qwen25_block.rs:1423-1478
    s = rich_shape(2)
    t = rich_map(s)
    ms = orc.Model(s, t, 16, threads=2)
    mc = orc.Model(s, t, 16, threads=3)
    assert ms.forward_token(2, 0) == 0 and mc.forward_token(2, 0) == 0
    prompt = [1, 3, 0, 4, 2]
    serial = _serial(ms, prompt, 1)
    assert mc.prefill(prompt) == 0
    assert fbits(mc.logits()) == fbits(serial)
    assert mc.cache_len() == ms.cache_len() == 6
    assert _kv_bits(mc, s, 6) == _kv_bits(ms, s, 6)
    rc1, o1 = ms.greedy_decode(3)
    rc2, o2 = mc.greedy_decode(3)
    assert rc1 == rc2 == 0 and list(o1) == list(o2)
    assert fbits(mc.logits()) == fbits(ms.logits())
    # batch tail: 33 tokens, one layer
    w = rich_shape(1)
    t1 = rich_map(w)
    toks = [i % 5 for i in range(33)]
    ms = orc.Model(w, t1, 40, threads=1)
    mc = orc.Model(w, t1, 40, threads=4)
    serial = _serial(ms, toks, 0)
    assert mc.prefill(toks) == 0
    assert fbits(mc.logits()) == fbits(serial) and mc.cache_len() == 33
    assert _kv_bits(mc, w, 33) == _kv_bits(ms, w, 33)


# -------------------------------------------------- bf16 KV cache mode ----
# The reference's cache is f32 (kv_cache.rs:93-94). The bf16 variant the
# long-context workload names rounds every K/V value to bf16 (nearest, ties
# to even) when it is stored, and the decode step's own row the same way, so
# attention always reads the values a bf16 slot holds.

def test_round_bf16_closed_forms(orc):
    r = lambda x: float(orc.round_bf16(np.float32(x)))
    for x in (1.0, -2.5, 0.0, 2.0 ** -126, 3.0 * 2.0 ** 100, 1.0 + 2.0 ** -7):
        assert r(x) == x  # exactly representable values survive
    assert r(1.0 + 2.0 ** -8) == 1.0                      # tie -> even (mantissa 0)
    assert r(1.0 + 3.0 * 2.0 ** -8) == 1.0 + 2.0 ** -6    # tie -> even (mantissa 2)
    assert r(-(1.0 + 3.0 * 2.0 ** -8)) == -(1.0 + 2.0 ** -6)
    assert r(1.0 + 2.0 ** -8 + 2.0 ** -20) == 1.0 + 2.0 ** -7  # above half
    assert r(1.0 + 2.0 ** -9) == 1.0                      # below half
    assert r(np.inf) == np.inf and r(-np.inf) == -np.inf
    assert math.isnan(r(np.nan))
    assert r(np.finfo(np.float32).max) == np.inf           # rounds past the largest bf16
    assert r(2.0 ** -140) == 0.0                           # a denormal below half the smallest bf16 step


def test_bf16_kv_closed_form(orc):
    # bf16_kv_fixture: v = [1 + 3 2^-8, 1 + 2^-9] rounds to [1 + 2^-6, 1].
    from model_fixtures import bf16_kv_fixture
    s, t = bf16_kv_fixture()
    v32 = [1.0 + 3.0 * 2.0 ** -8, 1.0 + 2.0 ** -9]
    v16 = [1.0 + 2.0 ** -6, 1.0]
    for bf16, v in ((False, v32), (True, v16)):
        m = orc.Model(s, t, 4, threads=1, kv_bf16=bf16)
        assert m.forward_token(0, 0) == 0
        # one position: the step's own row, as its slot holds it
        assert [float(x) for x in m.hidden()] == [1.0 + v[0], 1.0 + v[1]], bf16
        assert [float(x) for x in m.kv(0, 0, 0)[1]] == v
        # two positions weighted 1/2 each: the cached row and the step's row
        assert m.forward_token(0, 1) == 0
        assert [float(x) for x in m.hidden()] == [1.0 + v[0], 1.0 + v[1]], bf16
        # chunk prefill reads the chunk's rows back from the cache: the same
        p = orc.Model(s, t, 4, threads=1, kv_bf16=bf16)
        assert p.prefill([0, 0]) == 0
        assert fbits(p.hidden()) == fbits(m.hidden())
    m = orc.Model(s, t, 4, threads=1, kv_bf16=True)
    assert m.forward_token(0, 0) == 0
    assert orc.lib().orc_set_kv_bf16(m.h, 0) == 6  # only while the cache is empty


def test_bf16_kv_layer0_rows_are_rne_of_f32(orc):
    # Layer 0's K/V depend only on the prompt's embeddings, so the bf16 mode's
    # rows must be the f32 mode's rows rounded by an independent RNE.
    from model_fixtures import random_map, rne_bf16, shape_dict
    s = shape_dict(64, 4, 2, 16, 96, 50, 2, 1e-6)
    t = random_map(s, seed=5, std=0.3)
    f, b = orc.Model(s, t, 8, threads=2), orc.Model(s, t, 8, threads=2, kv_bf16=True)
    prompt = [3, 17, 41, 8, 22]
    assert f.prefill(prompt) == 0 and b.prefill(prompt) == 0
    assert b.forward_token(9, 5) == 0 and f.forward_token(9, 5) == 0
    changed = 0
    for h in range(2):
        for p in range(6):
            kf, vf = f.kv(0, h, p)
            kb, vb = b.kv(0, h, p)
            want_k = (rne_bf16(kf).astype(np.uint32) << 16).view(np.float32)
            want_v = (rne_bf16(vf).astype(np.uint32) << 16).view(np.float32)
            assert fbits(kb) == fbits(want_k) and fbits(vb) == fbits(want_v), (h, p)
            changed += int(np.sum(kb != kf)) + int(np.sum(vb != vf))
    assert changed > 0.9 * 2 * 6 * 2 * 16  # almost every value moved
    # later layers read rounded rows, so their results move too
    assert fbits(b.kv(1, 0, 5)[0]) != fbits((rne_bf16(f.kv(1, 0, 5)[0]).astype(np.uint32) << 16)
                                            .view(np.float32))


def test_bf16_kv_chunk_prefill_equals_serial(orc):
    # With every attention read taken from the cache's values, chunk prefill
    # and serial decode stay bit-identical in the bf16 mode too.
    s = rich_shape(2)
    t = rich_map(s)
    from model_fixtures import random_map, shape_dict
    for s, t in ((s, t), (shape_dict(32, 4, 2, 8, 48, 40, 2, 1e-6), None)):
        if t is None:
            t = random_map(s, seed=9, std=0.3)
        ms = orc.Model(s, t, 16, threads=2, kv_bf16=True)
        mc = orc.Model(s, t, 16, threads=3, kv_bf16=True)
        prompt = [1, 3, 0, 4, 2, 3, 1]
        serial = _serial(ms, prompt, 0)
        assert mc.prefill(prompt) == 0
        assert fbits(mc.logits()) == fbits(serial)
        assert _kv_bits(mc, s, 7) == _kv_bits(ms, s, 7)


# ----------------------------------------------------- attn_wire.rs ----

def _attn_model(orc, hidden, nq, nkv, d, proj, layers=1, max_seq=4):
    from model_fixtures import shape_dict
    s = shape_dict(hidden, nq, nkv, d, 2, 4, layers, 0.0)
    t = {"model.embed_tokens.weight": bits(np.zeros(4 * hidden), (4, hidden)),
         "model.norm.weight": bits(np.ones(hidden))}
    qd, kd = nq * d, nkv * d
    for l in range(layers):
        p = f"model.layers.{l}."
        t[p + "input_layernorm.weight"] = bits(np.ones(hidden))
        t[p + "post_attention_layernorm.weight"] = bits(np.ones(hidden))
        t[p + "self_attn.q_proj.weight"] = bits(proj["q_w"], (qd, hidden))
        t[p + "self_attn.q_proj.bias"] = bits(proj["q_b"])
        t[p + "self_attn.k_proj.weight"] = bits(proj["k_w"], (kd, hidden))
        t[p + "self_attn.k_proj.bias"] = bits(proj["k_b"])
        t[p + "self_attn.v_proj.weight"] = bits(proj["v_w"], (kd, hidden))
        t[p + "self_attn.v_proj.bias"] = bits(proj["v_b"])
        t[p + "self_attn.o_proj.weight"] = bits(proj["o_w"], (hidden, qd))
        for n in ("gate", "up"):
            t[p + f"mlp.{n}_proj.weight"] = bits(np.zeros(2 * hidden), (2, hidden))
        t[p + "mlp.down_proj.weight"] = bits(np.zeros(2 * hidden), (hidden, 2))
    return orc.Model(s, t, max_seq, threads=1)


def _matrix(rows, cols, columns):
    w = np.zeros((rows, cols), np.float32)
    for c, col in enumerate(columns):
        w[:, c] = col
    return w.ravel()


def test_attn_grouped_step(orc):
    # attn_wire.rs:450-517
    proj = dict(q_w=np.zeros(64), q_b=np.zeros(8), k_w=_matrix(4, 8, [[5, 6, 7, 8]]),
                k_b=np.zeros(4), v_w=_matrix(4, 8, [[1, 2, 3, 4]]), v_b=np.zeros(4),
                o_w=np.eye(8).ravel())
    m = _attn_model(orc, 8, 4, 2, 2, proj, max_seq=2)
    x = np.zeros(8, np.float32)
    x[0] = 1
    rc, r = m.attention_layer(0, 0, x, x)
    assert rc == 0 and list(r) == [2, 2, 1, 2, 3, 4, 3, 4] and m.cache_len() == 0
    assert list(m.kv(0, 0, 0)[0]) == [5, 6] and list(m.kv(0, 1, 0)[0]) == [7, 8]
    assert list(m.kv(0, 0, 0)[1]) == [1, 2] and list(m.kv(0, 1, 0)[1]) == [3, 4]


def test_attn_bias_after_gemv(orc):
    # attn_wire.rs:519-567
    proj = dict(q_w=np.zeros(16), q_b=[0.25, 0, 0, 0.5], k_w=_matrix(2, 4, [[2, 0]]),
                k_b=[1.0, 0.5], v_w=_matrix(2, 4, [[4, 0]]), v_b=[0.5, 1.0],
                o_w=np.eye(4).ravel())
    m = _attn_model(orc, 4, 2, 1, 2, proj, max_seq=2)
    x = np.array([1, 0, 0, 0], np.float32)
    rc, r = m.attention_layer(0, 0, x, x)
    assert list(r) == [5.5, 1.0, 4.5, 1.0]
    assert list(m.kv(0, 0, 0)[0]) == [3.0, 0.5] and list(m.kv(0, 0, 0)[1]) == [4.5, 1.0]


def test_attn_second_token_mix(orc):
    # attn_wire.rs:570-646
    proj = dict(q_w=np.zeros(16), q_b=np.zeros(4), k_w=np.zeros(16), k_b=np.zeros(4),
                v_w=_matrix(4, 4, [[4, 0, 0, 6], [0, 8, 2, 0]]), v_b=np.zeros(4),
                o_w=np.eye(4).ravel())
    m = _attn_model(orc, 4, 2, 2, 2, proj, max_seq=4)
    x0 = np.array([1, 0, 0, 0], np.float32)
    rc, r = m.attention_layer(0, 0, x0, x0)
    assert list(r) == [5, 0, 0, 6]
    assert m.advance() == 0
    x1 = np.array([0, 1, 0, 0], np.float32)
    rc, r = m.attention_layer(0, 1, x1, x1)
    assert list(r) == [2, 5, 1, 3] and m.cache_len() == 1
    assert list(m.kv(0, 0, 1)[1]) == [0, 8] and list(m.kv(0, 1, 1)[1]) == [2, 0]


def test_attn_rope_k_not_v(orc):
    # attn_wire.rs:648-704
    proj = dict(q_w=np.zeros(16), q_b=np.zeros(4), k_w=np.zeros(8), k_b=[1.0, 0.0],
                v_w=np.zeros(8), v_b=[4.0, 8.0], o_w=np.eye(4).ravel())
    m = _attn_model(orc, 4, 2, 1, 2, proj, max_seq=2)
    x = np.zeros(4, np.float32)
    m.attention_layer(0, 0, x, x)
    assert list(m.kv(0, 0, 0)[0]) == [1.0, 0.0]
    m.advance()
    m.attention_layer(0, 1, x, x)
    rot = orc.rope_f32_inplace([1.0, 0.0], 1, 2, THETA)[1]
    assert fbits(m.kv(0, 0, 1)[0]) == fbits(rot) and list(m.kv(0, 0, 1)[1]) == [4.0, 8.0]
