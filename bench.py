#!/usr/bin/env python3
"""Batch-1 BF16 token-loop benchmark on one MI355X.

Workload (one "step"): the reference's S1 scenario on a Qwen2.5-1.5B-shaped
random-init model (28 layers, hidden 1536, intermediate 8960, 12/2 heads,
head_dim 128, vocab 151936, tied head): KV cursor cleared, 128 seeded prompt
ids prefilled (MFMA GEMMs), then 128 greedy decode steps (one cooperative
kernel launch on the default path), batch 1, max_seq 256, f32 KV cache.

Prints one JSON line: value = decode tokens/s over the timed steps (weights
already resident in HBM), prefill tok/s beside it, the decode HBM-roofline
fraction (weights + KV bytes per token / 8 TB/s), the live roofline of the
dominant kernel (the cooperative decode kernel, timed with hipEvents on the
model's stream), and the CPU oracle timed on a bounded sample of the same
workload on the host cores.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
myos = importlib.import_module("an-operating-system-for-ai-models-and-tensor-inference_amd")

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
REF_CPU_DECODE_TOK_S = 15.4880  # reference S1 decode tok/s, 8 threads
METRIC = "decode tok/s + % HBM roofline, Qwen2.5-1.5B-shape bf16 bs=1; prefill tok/s"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))  # one GPU's share of the host


def weight_bytes(s) -> int:
    H, I, V, L = s.hidden, s.intermediate, s.vocab, s.num_layers
    Q, KD = s.num_q_heads * s.head_dim, s.num_kv_heads * s.head_dim
    per_layer = 2 * H + Q * H + Q + 2 * (KD * H + KD) + H * Q + 3 * I * H
    # bf16 bytes streamed per decode token: every layer, final norm, the head
    # (tied embed or lm_head), one embed row
    return 2 * (L * per_layer + H + V * H + H)


def kv_bytes_per_token(s, seq, kv_bytes) -> int:
    return s.num_layers * 2 * s.num_kv_heads * s.head_dim * seq * kv_bytes


def gemv_microbench(reps=5):
    """Isolated op-tier GEMV (bf16 W, f32 x, f32 accumulate) at the five
    decode shapes. One hipGraph per shape launches the GEMV once per weight
    copy; the copies total >= 512 MB (twice the last-level cache), so replays
    stream HBM. avg_us = replay time / launches (inter-kernel gaps included),
    from events on the replay stream."""
    import torch
    out = {}
    shapes = {"lm_head": (151936, 1536), "gate_or_up": (8960, 1536), "down": (1536, 8960),
              "q_or_o": (1536, 1536), "k_or_v": (256, 1536)}
    for name, (m, k) in shapes.items():
        nbytes = m * k * 2
        copies = max(2, -(-(512 << 20) // nbytes))
        gen = torch.Generator(device="cuda").manual_seed(m + k)
        ws = [(torch.randn(m, k, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
              for _ in range(copies)]
        x = torch.randn(k, device="cuda", generator=gen)
        y = torch.empty(m, device="cuda")
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            for w in ws:
                myos.gemv_bf16(y, w, x, m, k)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for w in ws:
                myos.gemv_bf16(y, w, x, m, k)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(ws))
        by = nbytes + k * 4 + m * 4
        out[name] = {"m": m, "k": k, "avg_us": round(us, 2), "GBps": round(by / us / 1e3, 1),
                     "frac_hbm": round(by / us / 1e3 / (HBM_PEAK / 1e9), 4),
                     "weight_copies": len(ws)}
        del graph, ws
        torch.cuda.empty_cache()
    return out


def cpu_baseline(path, shape, prompt, n_steps, gpu_ids):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    sd = dict(hidden=shape.hidden, num_q_heads=shape.num_q_heads,
              num_kv_heads=shape.num_kv_heads, head_dim=shape.head_dim,
              intermediate=shape.intermediate, vocab=shape.vocab,
              num_layers=shape.num_layers, rms_eps=np.float32(shape.rms_eps),
              rope_theta=np.float32(shape.rope_theta))
    t = oracle.load_safetensors_bits(path)
    cores = host_cores()
    out = {}
    for threads in sorted({cores, 8}, reverse=True):
        m = oracle.Model(sd, t, len(prompt) + n_steps, threads=threads)
        t0 = time.perf_counter()
        assert m.prefill(prompt) == 0
        t1 = time.perf_counter()
        rc, ids = m.greedy_decode(n_steps)
        t2 = time.perf_counter()
        assert rc == 0
        out[threads] = dict(prefill_s=t1 - t0, decode_s=t2 - t1, ids=[int(v) for v in ids])
        log(f"cpu oracle threads={threads}: prefill {len(prompt)} in {t1 - t0:.2f}s, "
            f"{n_steps} decode in {t2 - t1:.2f}s")
        del m
    ids = out[cores]["ids"]
    match = 0
    for a, b in zip(ids, gpu_ids):
        if a != b:
            break
        match += 1
    return cores, out, match


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--decode", type=int, default=128)
    ap.add_argument("--kv", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--weights", default=os.environ.get("MYOS_BENCH_WEIGHTS"))
    ap.add_argument("--cpu-decode-steps", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--decode-path", choices=["auto", "kernels", "persistent"], default="auto")
    ap.add_argument("--no-gemv-microbench", action="store_true")
    ap.add_argument("--shape", choices=["qwen2.5-1.5b", "qwen2.5-7b"], default="qwen2.5-1.5b",
                    help="model shape (the headline metric is quoted on qwen2.5-1.5b)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box here has one MI355X and this build has "
              f"no multi-GPU path (--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    if not args.no_gemv_microbench:
        # torch carries its own HIP runtime: it must initialise the device before
        # the library's runtime does (the microbench allocates through torch)
        import torch
        torch.cuda.init()
    is7b = args.shape == "qwen2.5-7b"
    shape = myos.preset(myos.SHAPE_QWEN25_7B if is7b else myos.SHAPE_QWEN25_1_5B)
    path = args.weights or ("/tmp/myos_bench/qwen25_7b_seed0.safetensors" if is7b
                            else "/tmp/myos_bench/qwen25_1_5b_seed0.safetensors")
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        log(f"writing random-init weights to {path}")
        t0 = time.perf_counter()
        myos.write_random_qwen25(path, shape, seed=0, std=0.02, threads=host_cores())
        log(f"weights written in {time.perf_counter() - t0:.1f}s")

    max_seq = args.prompt + args.decode
    kv = myos.KV_BF16 if args.kv == "bf16" else myos.KV_F32
    t0 = time.perf_counter()
    m = myos.Model.open(path, shape, kv, max_seq)
    t_load = time.perf_counter() - t0
    log(f"model resident in HBM in {t_load:.1f}s ({m.weight_bytes() / 1e9:.2f} GB weights)")
    if args.no_graph:
        m.set_graph(False)
    m.set_decode_mode({"auto": myos.DECODE_AUTO, "kernels": myos.DECODE_KERNELS,
                       "persistent": myos.DECODE_PERSISTENT}[args.decode_path])
    path_name = "persistent" if m.decode_path() == myos.DECODE_PERSISTENT else "kernels"
    log(f"decode path: {path_name}")
    rng = np.random.default_rng(2024)
    prompt = rng.integers(0, shape.vocab, args.prompt).astype(np.uint32)

    def step():
        m.cache_clear()
        a = time.perf_counter()
        m.prefill(prompt)
        b = time.perf_counter()
        ids = m.greedy_decode(args.decode)
        c = time.perf_counter()
        return b - a, c - b, ids, m.last_prefill_ms(), m.last_decode_ms()

    for i in range(args.warmup):
        step()
    log(f"{args.warmup} warmup steps done")
    tp = td = dp = dd = 0.0
    ids0 = None
    myos.lib().myos_stream_sync(None)
    w0 = time.perf_counter()
    for i in range(args.steps):
        a, b, ids, pms, dms = step()
        tp, td, dp, dd = tp + a, td + b, dp + pms, dd + dms
        ids0 = ids0 or ids
    myos.lib().myos_stream_sync(None)
    wall = time.perf_counter() - w0
    log(f"{args.steps} timed steps in {wall:.3f}s")

    decode_tok_s = args.steps * args.decode / td
    prefill_tok_s = args.steps * args.prompt / tp
    skv = 2 if kv == myos.KV_BF16 else 4
    wb = weight_bytes(shape)
    seqs = np.arange(args.prompt + 1, args.prompt + args.decode + 1)
    b_tok = wb + float(np.mean([kv_bytes_per_token(shape, int(q), skv) for q in seqs]))
    decode_frac = decode_tok_s * b_tok / HBM_PEAK

    # the dominant kernel: the cooperative decode kernel (one launch runs all
    # decode steps of a greedy_decode call) or, on the per-kernel path, the
    # fused gate/up GEMV; both timed with hipEvents on the model's stream
    kernels = {}
    for k, name in enumerate(myos.KERNEL_NAMES):
        ms = m.time_kernel(k, args.kernel_reps)
        by = m.kernel_bytes(k)
        kernels[name] = {"avg_us": round(ms * 1e3, 3), "bytes": int(by),
                         "GBps": round(by / (ms * 1e-3) / 1e9, 1)}
    log("per-kernel path: " + ", ".join(f"{n} {v['avg_us']}us {v['GBps']}GB/s"
                                        for n, v in kernels.items()))
    tpath = os.path.join(ROOT, "profiles", "decode_traffic_qwen25_1_5b.json")
    # the committed traffic figures are for the 1.5B shape with the f32 cache
    tinfo = (json.load(open(tpath))
             if os.path.exists(tpath) and kv == myos.KV_F32 and not is7b else {})
    if path_name == "persistent":
        launch_bytes = b_tok * args.decode
        launch_s = dd / args.steps * 1e-3
        achieved = launch_bytes / launch_s
        traffic = None
        t = tinfo.get("persistent_launch")
        if t and t.get("decode_steps") == args.decode and t.get("prompt_ids") == args.prompt:
            traffic = t["traffic_bytes"]
        roofline = {"bound": "hbm",
                    "kernel": f"decode_persistent_kernel (one launch: {args.decode} greedy "
                              f"decode steps)",
                    "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4), "traffic": traffic,
                    "algorithmic_bytes": int(launch_bytes),
                    "avg_launch_ms": round(dd / args.steps, 3)}
    else:
        dom = kernels["gate_up_swiglu"]
        achieved = dom["bytes"] / (dom["avg_us"] * 1e-6)
        roofline = {"bound": "hbm",
                    "kernel": "gate_up_swiglu (fused rmsnorm + gate/up GEMV + SwiGLU)",
                    "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                    "traffic": tinfo.get("traffic_bytes_per_launch", {}).get("gate_up_swiglu"),
                    "algorithmic_bytes": dom["bytes"]}
    m.close()

    micro = None if args.no_gemv_microbench else gemv_microbench()
    if micro:
        log("gemv microbench: " + ", ".join(f"{n} {v['avg_us']}us {v['GBps']}GB/s"
                                             for n, v in micro.items()))

    cpu = None
    if not args.no_cpu_baseline:
        n = args.cpu_decode_steps
        cores, res, match = cpu_baseline(path, shape, prompt, n, ids0)
        r = res[cores]
        cpu = {"value": round(n / r["decode_s"], 3), "unit": "tok/s", "cores": cores,
               "kind": "port",
               "sample": f"same weights file and 128 prompt ids: prefill 128 then {n} greedy "
                         f"decode steps on the C oracle (AVX2 GEMV, {cores} threads)",
               "prefill_tok_s": round(len(prompt) / r["prefill_s"], 2),
               "threads8_decode_tok_s": round(n / res[8]["decode_s"], 3) if 8 in res else None,
               "gpu_ids_equal_oracle_first_n": f"{match}/{n}"}

    line = {
        "metric": METRIC, "value": round(decode_tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None if is7b else round(decode_tok_s / REF_CPU_DECODE_TOK_S, 2),
        "dtype": "bf16", "data": "synthetic: random-init N(0,0.02) bf16 weights (seed 0), "
                                 "uniform prompt ids (seed 2024)",
        "config": {"workload": f"{'Qwen2.5-7B' if is7b else 'Qwen2.5-1.5B'}-shape S1: {args.prompt} prompt ids prefilled + "
                               f"{args.decode} greedy decode steps, batch 1",
                   "prompt_ids": args.prompt, "decode_steps": args.decode, "batch": 1,
                   "max_seq": max_seq, "kv_cache": args.kv, "accumulate": "f32",
                   "decode_path": path_name, "graph": not args.no_graph,
                   "parallelism": "single GPU"},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "decode_ms_per_token": round(td / (args.steps * args.decode) * 1e3, 4),
        "device_ms": {"prefill": round(dp / args.steps, 3), "decode": round(dd / args.steps, 3)},
        "decode_roofline": {"bytes_per_token": int(b_tok), "achieved_GBps":
                            round(decode_tok_s * b_tok / 1e9, 1), "peak_GBps": HBM_PEAK / 1e9,
                            "frac": round(decode_frac, 4)},
        "roofline": roofline, "per_kernel_path": kernels, "gemv_microbench": micro,
        "t_load_s": round(t_load, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
