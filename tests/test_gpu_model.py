"""Model-tier parity on the GPU against the oracle (model_core restated).

* the reference's block fixture: logits [1, 2, 0, -1], greedy ids [1, 1, 1, 1]
  (qwen25_block.rs:1011-1071, 1200-1221) -- exact in any summation order;
* the chunk-prefill fixture (rich_map, qwen25_block.rs:1423-1478): the GPU's
  MFMA prefill and its GEMV forward_token both agree with the oracle;
* seeded random small models, f32 and bf16 KV;
* prefill attention with and without key groups, for head_dim 32, 64, 128;
* the Qwen2.5-1.5B shape: prompt [0] + 4 greedy steps, and 128 prompt ids +
  teacher-forced decode, under the tolerance rule in parity.py.
"""
import importlib

import numpy as np
import pytest

import oracle
from model_fixtures import (block_fixture, random_map, rich_map, rich_shape, shape_dict,
                            write_safetensors)
from parity import assert_logits_parity, follow_ids, max_rel, top2_gap

myos = importlib.import_module("an-operating-system-for-ai-models-and-tensor-inference_amd")
pytestmark = pytest.mark.gpu


def to_block_shape(s, tied=True):
    return myos.make_shape(s["hidden"], s["num_q_heads"], s["num_kv_heads"], s["head_dim"],
                           s["intermediate"], s["vocab"], s["num_layers"],
                           rms_eps=float(s["rms_eps"]), rope_theta=float(s["rope_theta"]),
                           tied_head=tied)


def open_pair(tmp_path, s, t, max_seq, kv=myos.KV_F32, name="m.safetensors", tied=True):
    path = str(tmp_path / name)
    write_safetensors(path, t)
    g = myos.Model.open(path, to_block_shape(s, tied), kv, max_seq)
    # a bf16 cache is compared with the oracle's bf16 mode (K/V rounded to
    # nearest even when stored, the step's own row too)
    o = oracle.Model(s, t, max_seq, threads=4, kv_bf16=kv == myos.KV_BF16)
    return g, o


def test_block_fixture(tmp_path):
    s, t = block_fixture()
    g, o = open_pair(tmp_path, s, t, 8)
    g.forward_token(0, 0)
    assert list(g.logits()) == [1.0, 2.0, 0.0, -1.0]
    assert g.cache_len() == 1
    k, v = g.kv(0, 0, 0)
    assert list(k) == [0.0, 0.0] and list(v) == [1.0, 0.0]
    assert list(g.greedy_decode(4)) == [1, 1, 1, 1]
    assert g.cache_len() == 5
    assert list(g.kv(0, 0, 4)[1]) == [1.0, 0.0]
    # prefill path on a fresh model
    g2 = myos.Model.open(str(tmp_path / "m.safetensors"), to_block_shape(s), myos.KV_F32, 8)
    with pytest.raises(myos.MyosError) as e:
        g2.prefill([])
    assert e.value.kind == "Shape" and g2.cache_len() == 0
    g2.prefill([0])
    assert list(g2.logits()) == [1.0, 2.0, 0.0, -1.0]
    assert g2.greedy_decode(4) == [1, 1, 1, 1] and g2.cache_len() == 5
    for gm in (g, g2):
        gm.close()


def _both_paths(tmp_path, s, t, name, max_seq=4, tied=True):
    """The model on both forward paths: the per-kernel forward_token and the
    MFMA prefill."""
    path = str(tmp_path / name)
    write_safetensors(path, t)
    a = myos.Model.open(path, to_block_shape(s, tied), myos.KV_F32, max_seq)
    b = myos.Model.open(path, to_block_shape(s, tied), myos.KV_F32, max_seq)
    return a, b


def test_swiglu_residual_fixture(tmp_path, orc):
    # qwen25_block.rs:1074-1129, the only reference block vector with a
    # non-zero MLP: exact bits (every operand is small and exact), as pinned
    # on the oracle
    from model_fixtures import swiglu_residual_fixture
    s, t = swiglu_residual_fixture()
    o = orc.Model(s, t, 2, threads=1)
    assert o.forward_token(0, 0) == 0
    a, b = _both_paths(tmp_path, s, t, "swiglu.safetensors", 2)
    a.forward_token(0, 0)
    b.prefill([0])
    # (the MFMA prefill carries h = silu(1) in 16 significant bits: 1e-4)
    for m in (a, b):
        assert max_rel(m.logits(), o.logits()) < 1e-4
        assert max_rel(m.hidden(), o.hidden()) < 1e-4
        assert m.cache_len() == 1 and list(m.kv(0, 0, 0)[1]) == [1.0, 0.0]
        m.close()


def test_two_layer_fixture(tmp_path, orc):
    # qwen25_block.rs:1132-1197: per-layer V slots at one cursor, one advance
    # per token, on the forward_token, prefill and persistent paths
    from model_fixtures import two_layer_fixture
    s, t = two_layer_fixture()
    a, b = _both_paths(tmp_path, s, t, "two.safetensors", 4)
    a.forward_token(0, 0)
    b.prefill([0])
    for m in (a, b):
        assert list(m.logits()) == [1.0, 2.0, 0.0, -1.0] and m.cache_len() == 1
        assert list(m.kv(0, 0, 0)[1]) == [2.0, 0.0] and list(m.kv(1, 0, 0)[1]) == [0.0, 8.0]
        assert list(m.kv(0, 0, 1)[1]) == [0.0, 0.0] and list(m.kv(1, 0, 1)[1]) == [0.0, 0.0]
    a.forward_token(1, 1)
    b.decode_forced([1])
    o = orc.Model(s, t, 4, threads=1)
    assert o.forward_token(0, 0) == 0 and o.forward_token(1, 1) == 0
    for m in (a, b):
        assert m.cache_len() == 2
        assert list(m.kv(0, 0, 1)[1]) == [2.0, 0.0] and list(m.kv(1, 0, 1)[1]) == [0.0, 8.0]
        assert max_rel(m.logits(), o.logits()) < 1e-4
        assert int(np.argmax(m.logits())) == 1
        m.close()


def test_post_attention_norm_fixture(tmp_path, orc):
    # the closed-form fixture whose ln2 differs from ln1 (see the oracle pin
    # test_post_attention_norm_feeds_the_mlp)
    from model_fixtures import (bits, block_fixture_layer, fixture_embed_and_final,
                                fixture_shape)
    s = fixture_shape()
    t = fixture_embed_and_final((1.0, 0.5))
    block_fixture_layer(t, 0, [0.0] * 4, [1.0, 0.0], [1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0],
                        [1.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 1.0], [1.0, 0.0, 0.5, 0.0])
    t["model.layers.0.post_attention_layernorm.weight"] = bits([2.0, 0.0])
    o = orc.Model(s, t, 2, threads=1)
    assert o.forward_token(0, 0) == 0
    a, b = _both_paths(tmp_path, s, t, "norm2.safetensors", 2)
    a.forward_token(0, 0)
    b.prefill([0])
    for m in (a, b):
        assert max_rel(m.hidden(), o.hidden()) < 1e-4
        assert max_rel(m.logits(), o.logits()) < 1e-4
        m.close()


def test_untied_head_copy_equals_tied(tmp_path, orc):
    # an lm_head.weight equal to the embedding gives the tied head's logits;
    # a different one moves only the logits, and both match the oracle
    s = shape_dict(256, 4, 2, 64, 512, 1000, 2, 1e-6)
    t = random_map(s, seed=21, std=0.05)
    tu = dict(t)
    tu["lm_head.weight"] = np.array(t["model.embed_tokens.weight"], copy=True)
    td = dict(t)
    td["lm_head.weight"] = random_map(s, seed=22, std=0.05)["model.embed_tokens.weight"]
    prompt = [7, 300, 41, 999, 5]
    res = {}
    for name, tens, tied in (("tied", t, True), ("copy", tu, False), ("other", td, False)):
        path = str(tmp_path / f"{name}.safetensors")
        write_safetensors(path, tens)
        g = myos.Model.open(path, to_block_shape(s, tied), myos.KV_F32, 16)
        g.prefill(prompt)
        ids = g.greedy_decode(6)
        res[name] = (g.logits(), g.hidden(), ids)
        o = orc.Model(s, tens, 16, threads=2)
        assert o.prefill(prompt) == 0
        follow_ids(o, ids, name)
        assert_logits_parity(g.logits(), o.logits(), name)
        assert max_rel(g.logits(), o.logits()) < 1e-4
        g.close()
    assert np.array_equal(res["copy"][0], res["tied"][0]) and res["copy"][2] == res["tied"][2]
    assert not np.array_equal(res["other"][0], res["tied"][0])


def test_errors_do_not_advance(tmp_path):
    # qwen25_block.rs:1224-1300, 1481-1513
    s, t = block_fixture()
    path = str(tmp_path / "f.safetensors")
    write_safetensors(path, t)
    g = myos.Model.open(path, to_block_shape(s), myos.KV_F32, 2)
    for call, kind in ((lambda: g.forward_token(0, 1), "Position"),
                       (lambda: g.forward_token(9, 0), "TokenOutOfBounds"),
                       (lambda: g.prefill([0, 9]), "TokenOutOfBounds"),
                       (lambda: g.prefill([0, 0, 0]), "Full")):
        with pytest.raises(myos.MyosError) as e:
            call()
        assert e.value.kind == kind and g.cache_len() == 0
    assert list(g.logits()) == [0.0] * 4
    g.forward_token(0, 0)
    g.forward_token(1, 1)
    before = g.logits()
    with pytest.raises(myos.MyosError) as e:
        g.forward_token(1, 2)
    assert e.value.kind == "Full" and g.cache_len() == 2
    assert np.array_equal(g.logits(), before)
    with pytest.raises(myos.MyosError) as e:
        g.greedy_decode(3)
    assert e.value.kind == "Full" and e.value.partial == []
    g.close()


def _kv_all(m, s, n):
    out = []
    for l in range(s["num_layers"]):
        for h in range(s["num_kv_heads"]):
            for p in range(n):
                k, v = m.kv(l, h, p)
                out.append(np.concatenate([k, v]))
    return np.stack(out)


@pytest.mark.parametrize("graph", [True, False])
def test_rich_map_chunk_and_serial(tmp_path, graph):
    s = rich_shape(2)
    t = rich_map(s)
    g, o = open_pair(tmp_path, s, t, 16)
    g.set_graph(graph)
    gs = myos.Model.open(str(tmp_path / "m.safetensors"), to_block_shape(s), myos.KV_F32, 16)
    gs.set_graph(graph)
    for m in (g, gs):
        m.forward_token(2, 0)
    assert o.forward_token(2, 0) == 0
    prompt = [1, 3, 0, 4, 2]
    g.prefill(prompt)                      # chunk (MFMA)
    for i, tok in enumerate(prompt):       # serial (GEMV)
        gs.forward_token(tok, 1 + i)
    assert o.prefill(prompt) == 0
    ref = o.logits()
    for m in (g, gs):
        assert_logits_parity(m.logits(), ref, "rich_map")
        assert max_rel(m.hidden(), o.hidden()) < 1e-4
        assert max_rel(_kv_all(m, s, 6), _kv_all(o, s, 6)) < 1e-4
    rc, ids = o.greedy_decode(3)
    assert g.greedy_decode(3) == list(ids) == gs.greedy_decode(3)
    g.close()
    gs.close()


@pytest.mark.parametrize("kv", [myos.KV_F32, myos.KV_BF16])
@pytest.mark.parametrize("dims", [(256, 4, 2, 64, 512, 1000, 3), (128, 6, 1, 32, 384, 777, 2),
                                  (384, 12, 2, 32, 1000, 4099, 2)])
def test_random_small_models(tmp_path, kv, dims):
    s = shape_dict(*dims, 1e-6)
    t = random_map(s, seed=sum(dims), std=0.05)
    g, o = open_pair(tmp_path, s, t, 40, kv=kv)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, s["vocab"], 17)
    g.prefill(prompt)
    assert o.prefill(prompt) == 0
    # f32 cache: summation order only; bf16 cache: a cache value a few f32
    # ulps away from the oracle's may round to the neighbouring bf16 value
    tol = 1e-4 if kv == myos.KV_F32 else 2e-3
    assert max_rel(g.logits(), o.logits()) < tol
    assert max_rel(g.hidden(), o.hidden()) < tol
    # teacher-forced decode: both fed the oracle's greedy id
    for step in range(12):
        tok = oracle.greedy_token(o.logits())
        pos = o.cache_len()
        assert o.forward_token(tok, pos) == 0
        g.forward_token(tok, pos)
        assert max_rel(g.logits(), o.logits()) < tol, step
        assert_logits_parity(g.logits(), o.logits(), f"step {step}")
    g.close()


# Prefill attention runs four key groups per workgroup when the (q head,
# 16-query) grid is smaller than the 256 CUs and one group otherwise: each
# head_dim, at a prompt length on either side of that line (nq * ceil(M / 16)
# against 256), against the oracle.
@pytest.mark.parametrize("dims,m", [((384, 12, 2, 32, 1000, 4099, 2), 40),
                                    ((384, 12, 2, 32, 1000, 4099, 2), 400),
                                    ((256, 4, 2, 64, 512, 1000, 2), 40),
                                    ((256, 4, 2, 64, 512, 1000, 2), 1100),
                                    ((512, 4, 1, 128, 1536, 2048, 2), 40),
                                    ((512, 4, 1, 128, 1536, 2048, 2), 1100)])
def test_prefill_attention_key_groups(tmp_path, dims, m):
    s = shape_dict(*dims, 1e-6)
    t = random_map(s, seed=sum(dims) + m, std=0.05)
    g, o = open_pair(tmp_path, s, t, m + 8)
    prompt = np.random.default_rng(m).integers(0, s["vocab"], m)
    g.prefill(prompt)
    assert o.prefill(prompt) == 0
    assert max_rel(g.logits(), o.logits()) < 1e-4
    assert max_rel(g.hidden(), o.hidden()) < 1e-4
    assert_logits_parity(g.logits(), o.logits(), f"prefill of {m} ids")
    g.close()


# Gate/up over rows whose 128 x 256 tiles fill some rounds over the 256 CUs
# and leave a partial one: the N tiles of the whole rounds run in one launch,
# the rest in a tail launch on 128 x 128 tiles. N = 2 x 4352 = 34 wide tiles:
# 1100 rows (9 M tiles, 306 tiles) -> 28 of them, then 12 narrow N tiles x 9;
# 1000 rows (8 M tiles, 272) -> 32, then 4 x 8.
@pytest.mark.parametrize("m", [1000, 1100])
def test_gate_up_tail_launch(tmp_path, m):
    s = shape_dict(512, 4, 1, 128, 4352, 2048, 2, 1e-6)
    t = random_map(s, seed=m + 7, std=0.05)
    g, o = open_pair(tmp_path, s, t, m + 8)
    prompt = np.random.default_rng(m).integers(0, s["vocab"], m)
    g.prefill(prompt)
    assert o.prefill(prompt) == 0
    assert max_rel(g.logits(), o.logits()) < 1e-4
    assert max_rel(g.hidden(), o.hidden()) < 1e-4
    assert_logits_parity(g.logits(), o.logits(), f"prefill of {m} ids")
    g.close()


# Short prompts with head_dim 128 (33 to 128 ids, at most 256 keys) take the
# one-launch kernel that gives each wave its own key blocks; a prefill in
# chunks reaches it with a cache already holding rows (start position > 0),
# up to the 256-key limit. Each chunk's last logits and the final cache
# rows against the oracle's prefill of the same chunks.
@pytest.mark.parametrize("kv", [myos.KV_F32, myos.KV_BF16], ids=["f32_kv", "bf16_kv"])
@pytest.mark.parametrize("chunks", [(33,), (50, 70), (128, 128), (20, 100, 36)])
def test_short_prompt_attention_in_chunks(tmp_path, kv, chunks):
    s = shape_dict(512, 4, 1, 128, 1536, 2048, 2, 1e-6)
    t = random_map(s, seed=sum(chunks) + 11, std=0.05)
    n = sum(chunks)
    g, o = open_pair(tmp_path, s, t, n + 4, kv=kv)
    ids = np.random.default_rng(n).integers(0, s["vocab"], n)
    tol = 1e-4 if kv == myos.KV_F32 else 2e-3
    at = 0
    for c in chunks:
        g.prefill(ids[at:at + c])
        assert o.prefill(ids[at:at + c]) == 0
        at += c
        assert g.cache_len() == at
        assert max_rel(g.logits(), o.logits()) < tol, (chunks, at)
        assert max_rel(g.hidden(), o.hidden()) < tol, (chunks, at)
    # layer-1 cache rows: with a bf16 cache a row value a few f32 ulps from
    # the oracle's may round to the neighbouring bf16 value, one bf16 ulp
    # (2^-7 of the row's largest value at most)
    kv_tol = tol if kv == myos.KV_F32 else 2.0 ** -7
    for pos in (0, n // 2, n - 1):
        k, v = g.kv(1, 0, pos)
        ok, ov = o.kv(1, 0, pos)
        assert max_rel(k, ok) <= kv_tol and max_rel(v, ov) <= kv_tol, pos
    g.close()


# -------------------------------------------------- Qwen2.5-1.5B shape ----

@pytest.fixture(scope="module")
def qwen15(qwen15_path):
    s = shape_dict(1536, 12, 2, 128, 8960, 151936, 28, 1e-6)
    return qwen15_path, s, oracle.load_safetensors_bits(qwen15_path)


def test_qwen15_prompt0_four_steps(qwen15):
    # prompt [0], 4 greedy steps, batch 1 (max_seq 5)
    path, s, t = qwen15
    g = myos.Model.open(path, myos.preset(myos.SHAPE_QWEN25_1_5B), myos.KV_F32, 5)
    o = oracle.Model(s, t, 5, threads=16)
    g.prefill([0])
    assert o.prefill([0]) == 0
    assert_logits_parity(g.logits(), o.logits(), "prefill [0]")
    assert max_rel(g.hidden(), o.hidden()) < 1e-2
    ids_g = g.greedy_decode(4)
    rc, ids_o = o.greedy_decode(4)
    assert rc == 0
    assert ids_g == [int(v) for v in ids_o]
    assert_logits_parity(g.logits(), o.logits(), "after 4 steps")
    assert max_rel(g.hidden(), o.hidden()) < 1e-2
    g.close()


def test_qwen15_prefill128_teacher_forced(qwen15):
    # 128 seeded prompt ids prefilled on MFMA, then teacher-forced steps
    path, s, t = qwen15
    rng = np.random.default_rng(2024)
    prompt = rng.integers(0, 151936, 128)
    g = myos.Model.open(path, myos.preset(myos.SHAPE_QWEN25_1_5B), myos.KV_F32, 256)
    o = oracle.Model(s, t, 256, threads=16)
    g.prefill(prompt)
    assert o.prefill(prompt) == 0
    errs = [assert_logits_parity(g.logits(), o.logits(), "prefill 128")]
    assert max_rel(g.hidden(), o.hidden()) < 1e-2
    for step in range(6):
        tok = oracle.greedy_token(o.logits())
        pos = o.cache_len()
        assert o.forward_token(tok, pos) == 0
        g.forward_token(tok, pos)
        errs.append(assert_logits_parity(g.logits(), o.logits(), f"step {step}"))
        assert max_rel(g.hidden(), o.hidden()) < 1e-2
    k_g, v_g = g.kv(27, 1, 130)
    k_o, v_o = o.kv(27, 1, 130)
    assert max_rel(k_g, k_o) < 1e-2 and max_rel(v_g, v_o) < 1e-2
    print("max logits rel err per step:", ["%.2e" % e for e in errs])
    g.close()
