"""The oracle's pins must catch plausible mistakes in its composition.

Each case copies oracle/myos_oracle.c to a temporary directory, plants one
wiring mistake (MLP fed the pre-attention norm, a dropped residual, a layer's
K/V written to another layer's slots, the untied head ignored, RoPE on V, and
in the bf16 KV mode: the step's own row left unrounded, truncation for
round-to-nearest-even, V left unrounded),
compiles it with the oracle's own flags and runs the composition pins of
test_oracle_golden.py on it. At least one pin has to fail for every mistake.
CPU only: nothing here touches the product library or a GPU.
"""
import ctypes as C
import os
import shutil
import subprocess

import pytest

import oracle
import test_oracle_golden as golden

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(os.path.dirname(HERE), "oracle")

MUTATIONS = {
    "decode_mlp_reads_ln1": ("orc_rmsnorm_bf16_weight(m->normed, L->ln2, m->x",
                             "orc_rmsnorm_bf16_weight(m->normed, L->ln1, m->x"),
    "prefill_mlp_reads_ln1": ("L->ln2, X + i * H", "L->ln1, X + i * H"),
    "decode_mlp_residual_dropped": ("add_assign(m->x, m->mlp, H);", "(void)0;"),
    "kv_store_ignores_layer": ("size_t o = kv_off(m, layer, h, pos);\n    memcpy(m->kc + o, k",
                               "size_t o = kv_off(m, 0, h, pos);\n    memcpy(m->kc + o, k"),
    "untied_head_ignored": ("m->head = lm_head ? lm_head : embed;", "m->head = embed;"),
    "prefill_attends_layer0_cache": ("kv_pack(m, l, end);", "kv_pack(m, 0, end);"),
    "decode_rope_on_v": ("orc_rope_f32_inplace(m->k, kd,", "orc_rope_f32_inplace(m->v, kd,"),
    "bf16_kv_step_row_unrounded": ("    round_bf16_n(m->k, kd);\n    round_bf16_n(m->v, kd);\n", ""),
    "bf16_kv_truncates": ("u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;",
                          "u = u & 0xffff0000u;"),
    "bf16_kv_rounds_k_only": ("      round_bf16_n(m->vc + o, d);\n", ""),
}

PINS = [
    golden.test_block_fixture_forward,
    golden.test_swiglu_residual_changes_the_logits,
    golden.test_two_layers_advance_once_per_token,
    golden.test_post_attention_norm_feeds_the_mlp,
    golden.test_untied_head_copy_equals_tied,
    golden.test_chunk_prefill_equals_serial,
    golden.test_attn_rope_k_not_v,
    golden.test_round_bf16_closed_forms,
    golden.test_bf16_kv_closed_form,
    golden.test_bf16_kv_layer0_rows_are_rne_of_f32,
] + [lambda orc, d=d, s=s: golden.test_oracle_matches_textbook_forward(orc, d, s)
     for d, s in [((32, 4, 2, 8, 48, 40, 3), 1), ((64, 4, 4, 16, 80, 50, 4), 3)]]


def _build_mutant(tmp, old, new):
    src = open(os.path.join(SRC, "myos_oracle.c")).read()
    assert src.count(old) == 1, f"mutation anchor not unique: {old!r}"
    d = str(tmp)
    shutil.copy(os.path.join(SRC, "myos_oracle.h"), d)
    with open(os.path.join(d, "myos_oracle.c"), "w") as f:
        f.write(src.replace(old, new))
    so = os.path.join(d, "libmutant.so")
    subprocess.run(["gcc", "-O2", "-fPIC", "-std=gnu11", "-ffp-contract=off",
                    "-fno-fast-math", "-pthread", "-shared", "-o", so,
                    os.path.join(d, "myos_oracle.c"), "-lm"], check=True)
    lib = C.CDLL(so)
    oracle._declare(lib)
    return lib


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_pins_catch_mutation(tmp_path, monkeypatch, name):
    old, new = MUTATIONS[name]
    oracle.lib()
    monkeypatch.setattr(oracle, "_lib", _build_mutant(tmp_path, old, new))
    failed = []
    for pin in PINS:
        try:
            pin(oracle)
        except AssertionError:
            failed.append(getattr(pin, "__name__", "textbook"))
    assert failed, f"no pin caught the mutation {name}"


def test_unmutated_copy_passes_every_pin(tmp_path, monkeypatch):
    # the harness itself: the same build recipe without a mutation passes
    oracle.lib()
    monkeypatch.setattr(oracle, "_lib", _build_mutant(tmp_path, "int orc_kv_advance(", "int orc_kv_advance("))
    for pin in PINS:
        pin(oracle)
