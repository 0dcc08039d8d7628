#!/usr/bin/env python3
"""Writes the golden fixtures of the long-context and 7B parity tests.

The oracle (oracle/, the CPU restatement of the reference's token loop)
cannot run these workloads inside a GPU test in reasonable time (a 2048-id
prefill is minutes of serial attention on the CPU), so this script runs it
once, in the development container, and stores what the GPU tests compare
against:

* qwen25_1_5b_long.npz -- Qwen2.5-1.5B shape, random-init seed 0 (the
  bench's weights), 2048 seeded uniform prompt ids prefilled, then 256
  greedy decode steps (max_seq 2304), f32 KV cache;
* qwen25_1_5b_long_bf16kv.npz -- the same workload with the bf16 KV cache:
  the oracle's bf16 mode rounds every K/V value to bf16 (nearest, ties to
  even) when it is stored and the decode step's own row the same way;
* qwen25_7b_s1.npz -- Qwen2.5-7B shape (untied lm_head), seed 0, 128
  seeded prompt ids, then 128 greedy steps (greedy_decode,
  qwen25_block.rs:765-780).

Each holds the prompt, the logits / final hidden / normed vector after the
prefill and after the last step, every step's greedy id with its top-1 /
top-2 gap and its 8 largest logits (index, value), sampled KV rows, and a
sampled fingerprint of the weights file so a test can check it regenerated
the same bytes. Inputs come from the library's seeded writer
(myos_write_random_qwen25); every expected value comes from the oracle.

usage: python tests/golden/make_fixtures.py [long|long_bf16|7b|all] [--threads N]
"""
from __future__ import annotations

import argparse
import hashlib
import importlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402
from model_fixtures import shape_dict  # noqa: E402

myos = importlib.import_module("an-operating-system-for-ai-models-and-tensor-inference_amd")

PROMPT_SEED = 2024
TOPK = 8


def file_fingerprint(path: str) -> str:
    """sha256 over the SafeTensors header and 4 KiB every 64 MiB of payload."""
    h = hashlib.sha256()
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        f.seek(0)
        h.update(f.read(8 + n))
        for off in range(8 + n, size, 64 << 20):
            f.seek(off)
            h.update(f.read(4096))
    h.update(str(size).encode())
    return h.hexdigest()


def topk(lg):
    idx = np.argsort(-lg.astype(np.float64), kind="stable")[:TOPK]
    return idx.astype(np.uint32), lg[idx].astype(np.float32)


def run(name, preset, n_prompt, n_steps, kv_points, threads, workdir, kv_bf16=False,
        weights=None):
    shape = myos.preset(preset)
    path = os.path.join(workdir, f"{weights or name}_seed0.safetensors")
    if not os.path.exists(path):
        t0 = time.time()
        myos.write_random_qwen25(path, shape, seed=0, std=0.02, threads=threads)
        print(f"[{name}] wrote {path} in {time.time() - t0:.0f}s", flush=True)
    s = shape_dict(shape.hidden, shape.num_q_heads, shape.num_kv_heads, shape.head_dim,
                   shape.intermediate, shape.vocab, shape.num_layers, shape.rms_eps,
                   shape.rope_theta)
    t = oracle.load_safetensors_bits(path)
    max_seq = n_prompt + n_steps
    m = oracle.Model(s, t, max_seq, threads=threads, kv_bf16=kv_bf16)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, shape.vocab, n_prompt).astype(np.uint32)
    t0 = time.time()
    assert m.prefill(prompt) == 0
    print(f"[{name}] prefill {n_prompt} in {time.time() - t0:.0f}s", flush=True)
    out = dict(prompt=prompt, prefill_logits=m.logits(), prefill_hidden=m.hidden(),
               prefill_normed=m.normed())
    ids, gaps, tki, tkv = [], [], [], []
    t0 = time.time()
    for step in range(n_steps):
        lg = m.logits()
        tok = int(oracle.greedy_token(lg))
        i, v = topk(lg)
        assert i[0] == tok
        ids.append(tok)
        gaps.append(float(np.float64(v[0]) - np.float64(v[1])))
        tki.append(i)
        tkv.append(v)
        assert m.forward_token(tok, m.cache_len()) == 0
        if step % 32 == 31:
            print(f"[{name}] {step + 1} steps, {time.time() - t0:.0f}s", flush=True)
    out.update(ids=np.array(ids, np.uint32), gaps=np.array(gaps, np.float64),
               topk_idx=np.stack(tki), topk_val=np.stack(tkv), final_logits=m.logits(),
               final_hidden=m.hidden(), final_normed=m.normed())
    layers, heads, positions = kv_points
    kv = np.zeros((len(layers), len(heads), len(positions), 2, shape.head_dim), np.float32)
    for a, l in enumerate(layers):
        for b, h in enumerate(heads):
            for c, p in enumerate(positions):
                kv[a, b, c, 0], kv[a, b, c, 1] = m.kv(l, h, p)
    out.update(kv=kv, kv_layers=np.array(layers), kv_heads=np.array(heads),
               kv_positions=np.array(positions), max_seq=np.array(max_seq),
               kv_bf16=np.array(bool(kv_bf16)),
               weights_fingerprint=np.array(file_fingerprint(path)),
               shape=np.array([shape.hidden, shape.num_q_heads, shape.num_kv_heads,
                               shape.head_dim, shape.intermediate, shape.vocab,
                               shape.num_layers, shape.tied_head]))
    dst = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(dst, **out)
    print(f"[{name}] wrote {dst} ({os.path.getsize(dst) / 1e6:.2f} MB); ids {ids[:8]}..., "
          f"min gap {min(gaps):.3e}", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("which", nargs="?", default="all", choices=["long", "long_bf16", "7b", "all"])
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 8)
    ap.add_argument("--workdir", default="/tmp/myos_fixtures")
    a = ap.parse_args()
    os.makedirs(a.workdir, exist_ok=True)
    if a.which in ("long", "all"):
        run("qwen25_1_5b_long", myos.SHAPE_QWEN25_1_5B, 2048, 256,
            ([0, 13, 27], [0, 1], [0, 1023, 2047, 2048, 2175, 2303]), a.threads, a.workdir)
    if a.which in ("long_bf16", "all"):
        run("qwen25_1_5b_long_bf16kv", myos.SHAPE_QWEN25_1_5B, 2048, 256,
            ([0, 13, 27], [0, 1], [0, 1023, 2047, 2048, 2175, 2303]), a.threads, a.workdir,
            kv_bf16=True, weights="qwen25_1_5b_long")
    if a.which in ("7b", "all"):
        run("qwen25_7b_s1", myos.SHAPE_QWEN25_7B, 128, 128,
            ([0, 13, 27], [0, 3], [0, 127, 128, 191, 255]), a.threads, a.workdir)


if __name__ == "__main__":
    main()
