#!/usr/bin/env python3
"""Batch-1 BF16 token-loop benchmark on one MI355X.

Workload (one "step"): the reference's S1 scenario on a Qwen2.5-1.5B-shaped
random-init model (28 layers, hidden 1536, intermediate 8960, 12/2 heads,
head_dim 128, vocab 151936, tied head): KV cursor cleared, 128 seeded prompt
ids prefilled (MFMA GEMMs), then 128 greedy decode steps (one cooperative
kernel launch on the default path), batch 1, max_seq 256, f32 KV cache.

Prints one JSON line: value = decode tokens/s over the timed steps (weights
already resident in HBM), prefill tok/s beside it, the decode and prefill
HBM-roofline fractions (bytes per token / 8 TB/s), the live roofline of the
dominant kernel (the cooperative decode kernel, timed with hipEvents on the
model's stream), the parity of the timed run against the oracle, the
fresh-process W/R medians of the CLI's arena harness, and the CPU oracle on
the same workload (medians, host core count and 8 threads). The host-only
legs (oracle, arena children) run before this process touches the GPU.
After the timed region, each on its own model: a 2048-id prefill alone, the
long-context workload (2048 ids + 256 greedy steps, bf16 cache) and the
7B shape's S1 (128 + 128).
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
MFMA_BF16_PEAK = 2.5e15  # MI355X dense bf16 MFMA, FLOP/s
REF_CPU_DECODE_TOK_S = 15.4880  # reference S1 decode tok/s, 8 threads (arena/phase1-scoreboard.md:28)
METRIC = "decode tok/s + % HBM roofline, Qwen2.5-1.5B-shape bf16 bs=1; prefill tok/s"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_nproc() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def host_cores() -> int:
    # the reference caps --threads at 64 (gemv_bf16_kernel.rs:34,
    # main.rs:416-424); the benchmark hosts allot 16 host cores per GPU
    return max(1, min(16, host_nproc(), 64))


def weight_bytes(s) -> int:
    H, I, V, L = s.hidden, s.intermediate, s.vocab, s.num_layers
    Q, KD = s.num_q_heads * s.head_dim, s.num_kv_heads * s.head_dim
    per_layer = 2 * H + Q * H + Q + 2 * (KD * H + KD) + H * Q + 3 * I * H
    # bf16 bytes streamed per decode token: every layer, final norm, the head
    # (tied embed or lm_head), one embed row
    return 2 * (L * per_layer + H + V * H + H)


def kv_bytes_per_token(s, seq, kv_bytes) -> int:
    return s.num_layers * 2 * s.num_kv_heads * s.head_dim * seq * kv_bytes


def prefill_flops(s, n) -> float:
    """Algorithmic FLOPs of prefilling n ids from an empty cache: every
    projection as a GEMM over the n rows, causal attention (q.k and p.v over
    the keys each query sees) and the head for the last id only."""
    qd, kvd = s.num_q_heads * s.head_dim, s.num_kv_heads * s.head_dim
    per_row = s.hidden * (qd + 2 * kvd) + qd * s.hidden + 3 * s.hidden * s.intermediate
    attn = 2.0 * s.num_q_heads * s.head_dim * (n * (n + 1) / 2.0)
    return s.num_layers * (2.0 * n * per_row + 2.0 * attn) + 2.0 * s.vocab * s.hidden


def prefill_leg(path, shape, kv, n, reps=3):
    """The MFMA prefill alone on n seeded ids (one warm-up, median of reps
    device times), from an empty cache of max_seq n."""
    ids = np.random.default_rng(2048).integers(0, shape.vocab, n).astype(np.uint32)
    ms = []
    with myos.Model.open(path, shape, kv, n) as g:
        for r in range(reps + 1):
            g.cache_clear()
            g.prefill(ids)
            if r:
                ms.append(g.last_prefill_ms())
    t = float(np.median(ms))
    fl = prefill_flops(shape, n)
    return {"prompt_ids": n, "device_ms": round(t, 3), "tok_s": round(n / (t * 1e-3), 1),
            "flops_alg": fl, "mfma_frac_alg": round(fl / (t * 1e-3) / MFMA_BF16_PEAK, 4),
            "runs": [round(x, 3) for x in ms]}


def committed_traffic(is7b, path_name, n_prompt, n_decode, kv_name):
    """The committed rocprof HBM traffic of one cooperative decode launch of
    this workload (profiles/decode_traffic_*.json, FETCH_SIZE + WRITE_SIZE
    scaled by a copy-kernel calibration), or (None, None)."""
    tpath = os.path.join(ROOT, "profiles", f"decode_traffic_qwen25_{'7b' if is7b else '1_5b'}.json")
    if not os.path.exists(tpath):
        return None, None
    for key, t in json.load(open(tpath)).items():
        if (key.startswith(f"{path_name}_launch") and isinstance(t, dict)
                and t.get("prompt_ids") == n_prompt and t.get("decode_steps") == n_decode
                and t.get("kv_cache", "f32") == kv_name):
            return t["traffic_bytes"], t["source"]
    return None, None


def decode_leg(path, shape, kv, n_prompt, n_decode, is7b, reps=3):
    """Another workload on its own model, outside the timed region: n_prompt
    seeded ids prefilled, then n_decode greedy steps on the default decode
    path; one warm-up, the median device times of reps runs and the decode
    roofline at each step's cache length."""
    prompt = bench_prompt(shape, n_prompt)
    skv = 2 if kv == myos.KV_BF16 else 4
    pre, dec, ids = [], [], None
    with myos.Model.open(path, shape, kv, n_prompt + n_decode) as g:
        pname = {myos.DECODE_PERSISTENT: "persistent", myos.DECODE_STREAMED: "streamed",
                 myos.DECODE_KERNELS: "kernels"}[g.decode_path()]
        for r in range(reps + 1):
            g.cache_clear()
            g.prefill(prompt)
            out = g.greedy_decode(n_decode)
            if r:
                pre.append(g.last_prefill_ms())
                dec.append(g.last_decode_ms())
                ids = ids or out
    d = float(np.median(dec))
    seqs = np.arange(n_prompt + 1, n_prompt + n_decode + 1)
    b_tok = weight_bytes(shape) + float(np.mean([kv_bytes_per_token(shape, int(q), skv) for q in seqs]))
    tok_s = n_decode / (d * 1e-3)
    kv_name = "bf16" if skv == 2 else "f32"
    traffic, tsrc = committed_traffic(is7b, pname, n_prompt, n_decode, kv_name)
    import hashlib
    return {"workload": workload_name(is7b, n_prompt, n_decode, kv_name),
            "decode_path": pname, "decode_tok_s": round(tok_s, 2),
            "device_ms": {"prefill": round(float(np.median(pre)), 3), "decode": round(d, 3)},
            "decode_roofline": {"bytes_per_token": int(b_tok),
                                "achieved_GBps": round(tok_s * b_tok / 1e9, 1),
                                "frac": round(tok_s * b_tok / HBM_PEAK, 4),
                                "launch_traffic": traffic, "launch_algorithmic_bytes": int(b_tok * n_decode),
                                "traffic_source": tsrc and f"{tsrc} (not measured in this run)"},
            "runs_decode_ms": [round(x, 3) for x in dec],
            "ids_sha1": hashlib.sha1(np.asarray(ids, np.uint32).tobytes()).hexdigest()[:16]}


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


def _oracle_shape(shape):
    return dict(hidden=shape.hidden, num_q_heads=shape.num_q_heads,
                num_kv_heads=shape.num_kv_heads, head_dim=shape.head_dim,
                intermediate=shape.intermediate, vocab=shape.vocab,
                num_layers=shape.num_layers, rms_eps=np.float32(shape.rms_eps),
                rope_theta=np.float32(shape.rope_theta))


def cpu_baseline(path, shape, prompt, n_steps, repeats):
    """The oracle (the C restatement of the reference's CPU path: AVX2 32-row
    GEMV over a row-span thread pool, serial attention) on the same weights
    and prompt: prefill, then n_steps greedy steps, `repeats` scored runs
    after one short warm-up, at the host core count and at 8 threads.
    Medians (meter.rs:86-98); also each step's greedy id and top-1 / top-2
    gap and the final logits, for the parity fields of the bench line."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    sd = _oracle_shape(shape)
    t = oracle.load_safetensors_bits(path)
    out = {}
    ref = None
    for threads in sorted({host_cores(), 8}, reverse=True):
        m = oracle.Model(sd, t, len(prompt) + n_steps, threads=threads)
        assert m.prefill(prompt[:8]) == 0  # warm-up: the pool and the weight pages
        pre, dec = [], []
        for r in range(repeats):
            m = oracle.Model(sd, t, len(prompt) + n_steps, threads=threads)
            t0 = time.perf_counter()
            assert m.prefill(prompt) == 0
            t1 = time.perf_counter()
            ids, gaps = [], []
            for _ in range(n_steps):
                lg = m.logits()
                tok = int(oracle.greedy_token(lg))
                if ref is None:
                    srt = np.sort(lg.astype(np.float64))
                    gaps.append(float(srt[-1] - srt[-2]))
                ids.append(tok)
                assert m.forward_token(tok, m.cache_len()) == 0
            t2 = time.perf_counter()
            pre.append(t1 - t0)
            dec.append(t2 - t1)
            if ref is None:
                ref = dict(ids=ids, gaps=gaps, final_logits=m.logits())
            log(f"cpu oracle threads={threads} run {r + 1}/{repeats}: prefill {len(prompt)} in "
                f"{t1 - t0:.2f}s, {n_steps} decode in {t2 - t1:.2f}s")
        out[threads] = dict(prefill_s=float(np.median(pre)), decode_s=float(np.median(dec)))
        del m
    return out, ref


def run_arena(path, shape_name, prompt, ref_ids, n_steps, kv, warmup, repeats):
    """The CLI's --arena-s1 harness (W warm-up + R scored fresh processes,
    medians, DET / CORRECT gates against the oracle's ids), started before
    this process touches the GPU."""
    import subprocess
    import tempfile
    d = tempfile.mkdtemp(prefix="myos_arena_")
    pp, rp = os.path.join(d, "prompt.txt"), os.path.join(d, "ref.txt")
    with open(pp, "w") as f:
        f.write(" ".join(str(int(v)) for v in prompt) + "\n")
    with open(rp, "w") as f:
        f.write(" ".join(str(int(v)) for v in ref_ids) + "\n")
    cmd = [myos.CLI_PATH, "--arena-s1", "--weights", path, "--prompt-ids", pp, "--ref-ids", rp,
           "--steps", str(n_steps), "--warmup", str(warmup), "--repeats", str(repeats),
           "--model-shape", shape_name, "--kv", kv, "--fingerprint-dir", os.path.join(d, "run")]
    t0 = time.perf_counter()
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    log(f"arena W={warmup} R={repeats} in {time.perf_counter() - t0:.1f}s: "
        f"{r.stdout.strip().splitlines()[0] if r.stdout.strip() else r.stderr[-300:]}")
    agg_path = os.path.join(d, "run", "metrics.json")
    if not os.path.exists(agg_path):
        return {"error": (r.stderr or r.stdout)[-400:], "exit": r.returncode}
    agg = json.load(open(agg_path))
    return {"W": agg["W"], "R": agg["R"], "det": agg["det"], "correct": agg["CORRECT"],
            "median": agg["median"], "min": agg["min"], "max": agg["max"],
            "exit": r.returncode, "run_dir": os.path.join(d, "run")}


def workload_name(is7b, n_prompt, n_decode, kv):
    """The run's workload by its own name: S1 is 128 + 128, the long-context
    workload 2048 + 256; anything else is named by its sizes only."""
    shape = "Qwen2.5-7B" if is7b else "Qwen2.5-1.5B"
    name = {(128, 128): " S1", (2048, 256): " long-context"}.get((n_prompt, n_decode), "")
    return (f"{shape}-shape{name}: {n_prompt} prompt ids prefilled + {n_decode} greedy decode "
            f"steps, batch 1, {kv} KV cache")


def bench_prompt(shape, n):
    return np.random.default_rng(2024).integers(0, shape.vocab, n).astype(np.uint32)


PATH_7B = "/tmp/myos_bench/qwen25_7b_seed0.safetensors"


def other_legs(args, is7b):
    """The default S1 run also measures the long-context workload (2048 + 256,
    bf16 cache) and the 7B shape's S1, each on its own model after the timed
    region."""
    return not is7b and args.prompt == 128 and args.decode == 128 and args.kv == "f32"


def host_legs(args, is7b, path, n_cpu):
    """The child process of the host-only legs: writes the weights file if it
    is missing, then runs the CPU baseline and the arena; results go to
    <dir>/host.json and <dir>/ref_logits.npy."""
    shape = myos.preset(myos.SHAPE_QWEN25_7B if is7b else myos.SHAPE_QWEN25_1_5B)
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        log(f"writing random-init weights to {path}")
        t0 = time.perf_counter()
        myos.write_random_qwen25(path, shape, seed=0, std=0.02, threads=host_cores())
        log(f"weights written in {time.perf_counter() - t0:.1f}s")
    if other_legs(args, is7b) and not args.no_7b and not os.path.exists(PATH_7B):
        log(f"writing random-init 7B-shape weights to {PATH_7B}")
        t0 = time.perf_counter()
        try:
            myos.write_random_qwen25(PATH_7B, myos.preset(myos.SHAPE_QWEN25_7B), seed=0, std=0.02,
                                     threads=host_cores())
            log(f"7B weights written in {time.perf_counter() - t0:.1f}s")
        except Exception as e:  # e.g. no room for 15 GB: the 7B leg reports the error
            log(f"7B weights not written: {e}")
            if os.path.exists(PATH_7B):
                os.remove(PATH_7B)
    prompt = bench_prompt(shape, args.prompt)
    cpu_res, ref = None, None
    if not args.no_cpu_baseline:
        cpu_res, ref = cpu_baseline(path, shape, prompt, n_cpu, args.cpu_repeats)
    arena = None
    if not args.no_arena and ref is not None and n_cpu == args.decode:
        arena = run_arena(path, "7b" if is7b else "1.5b", prompt, ref["ids"], args.decode,
                          args.kv, args.arena_warmup, args.arena_repeats)
    if ref is not None:
        np.save(os.path.join(args.host_legs, "ref_logits.npy"), ref.pop("final_logits"))
    with open(os.path.join(args.host_legs, "host.json"), "w") as f:
        json.dump({"cpu": cpu_res, "ref": ref, "arena": arena}, f)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--decode", type=int, default=128)
    ap.add_argument("--kv", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--weights", default=os.environ.get("MYOS_BENCH_WEIGHTS"))
    ap.add_argument("--cpu-decode-steps", type=int, default=None,
                    help="greedy steps of the CPU baseline (default: all --decode steps)")
    ap.add_argument("--cpu-repeats", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--arena-warmup", type=int, default=3)
    ap.add_argument("--arena-repeats", type=int, default=5)
    ap.add_argument("--no-arena", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--decode-path", choices=["auto", "kernels", "persistent", "streamed"],
                    default="auto")
    ap.add_argument("--no-gemv-microbench", action="store_true")
    ap.add_argument("--no-prefill-2048", action="store_true",
                    help="skip the 2048-id prefill-only leg")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip the 2048 + 256 bf16-cache decode leg")
    ap.add_argument("--no-7b", action="store_true", help="skip the 7B-shape S1 decode leg")
    ap.add_argument("--shape", choices=["qwen2.5-1.5b", "qwen2.5-7b"], default="qwen2.5-1.5b",
                    help="model shape (the headline metric is quoted on qwen2.5-1.5b)")
    ap.add_argument("--host-legs", metavar="DIR", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box here has one MI355X and this build has "
              f"no multi-GPU path (--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    is7b = args.shape == "qwen2.5-7b"
    path = args.weights or (PATH_7B if is7b else "/tmp/myos_bench/qwen25_1_5b_seed0.safetensors")
    n_cpu = args.cpu_decode_steps or args.decode
    if args.host_legs:
        host_legs(args, is7b, path, n_cpu)
        return

    # The host-only legs run in a child process before this one touches the
    # GPU: the weights file (if missing), the CPU baseline (the oracle) and the
    # fresh-process arena runs. This process then initialises torch's HIP
    # runtime before it loads the library (the microbench allocates through
    # torch, whose runtime has to come up first).
    import subprocess
    import tempfile
    hdir = tempfile.mkdtemp(prefix="myos_bench_host_")
    cmd = [sys.executable, "-u", os.path.abspath(__file__), "--host-legs", hdir] + sys.argv[1:]
    t0 = time.perf_counter()
    r = subprocess.run(cmd)
    if r.returncode != 0:
        log(f"host legs failed (exit {r.returncode})")
        sys.exit(r.returncode)
    host = json.load(open(os.path.join(hdir, "host.json")))
    log(f"host legs done in {time.perf_counter() - t0:.1f}s")
    cpu_res = {int(k): v for k, v in host["cpu"].items()} if host["cpu"] else None
    ref = host["ref"]
    if ref is not None:
        ref["final_logits"] = np.load(os.path.join(hdir, "ref_logits.npy"))
    arena = host["arena"]

    if not args.no_gemv_microbench:
        import torch
        torch.cuda.init()
    shape = myos.preset(myos.SHAPE_QWEN25_7B if is7b else myos.SHAPE_QWEN25_1_5B)
    prompt = bench_prompt(shape, args.prompt)
    max_seq = args.prompt + args.decode
    kv = myos.KV_BF16 if args.kv == "bf16" else myos.KV_F32
    t0 = time.perf_counter()
    m = myos.Model.open(path, shape, kv, max_seq)
    t_load = time.perf_counter() - t0
    log(f"model resident in HBM in {t_load:.1f}s ({m.weight_bytes() / 1e9:.2f} GB weights)")
    if args.no_graph:
        m.set_graph(False)
    m.set_decode_mode({"auto": myos.DECODE_AUTO, "kernels": myos.DECODE_KERNELS,
                       "persistent": myos.DECODE_PERSISTENT,
                       "streamed": myos.DECODE_STREAMED}[args.decode_path])
    path_name = {myos.DECODE_PERSISTENT: "persistent", myos.DECODE_STREAMED: "streamed",
                 myos.DECODE_KERNELS: "kernels"}[m.decode_path()]
    log(f"decode path: {path_name}")

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
    # prefill: every projection weight byte once, the head once (last id), and
    # the cache rows written
    prefill_bytes = wb - 2 * shape.hidden + kv_bytes_per_token(shape, args.prompt, skv)
    prefill_ms = dp / args.steps
    pf_roof = {"bound": "hbm", "bytes": int(prefill_bytes), "avg_ms": round(prefill_ms, 4),
               "achieved_GBps": round(prefill_bytes / (prefill_ms * 1e-3) / 1e9, 1),
               "frac": round(prefill_bytes / (prefill_ms * 1e-3) / HBM_PEAK, 4)}

    # parity of the timed run: the GPU ids under the tolerance rule against
    # the oracle's (each step's top-1 / top-2 gap), then both decode paths
    # teacher-forced with the oracle's ids against the oracle's final logits:
    # the cooperative kernel multiplies gate/up, the down partials and the
    # head with v_dot2 over the activations split into bf16 hi + lo (16
    # significant bits); the per-kernel path keeps f32 activations
    parity = None
    if ref is not None and n_cpu == args.decode:
        agree, first_div = 0, None
        for i, (a, b) in enumerate(zip(ids0, ref["ids"])):
            if a != b:
                first_div = {"step": i, "oracle_gap": ref["gaps"][i]}
                break
            agree += 1
        o_lg = ref["final_logits"]
        rel = {}
        for name, mode in (("persistent", myos.DECODE_PERSISTENT),
                           ("streamed", myos.DECODE_STREAMED),
                           ("kernels", myos.DECODE_KERNELS)):
            try:
                m.set_decode_mode(mode)
            except myos.MyosError:
                continue
            m.cache_clear()
            m.prefill(prompt)
            m.decode_forced(ref["ids"])
            g = m.logits().astype(np.float64)
            rel[name] = float(np.max(np.abs(g - o_lg)) / np.max(np.abs(o_lg)))
        m.set_decode_mode(myos.DECODE_AUTO)
        parity = {"ids_equal_oracle_prefix": f"{agree}/{args.decode}",
                  "first_divergence": first_div,
                  "min_oracle_top2_gap": round(float(min(ref["gaps"])), 6),
                  "teacher_forced_final_logits_max_rel_err_vs_oracle": rel}

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
    tpath = os.path.join(ROOT, "profiles",
                         f"decode_traffic_qwen25_{'7b' if is7b else '1_5b'}.json")
    # the committed per-kernel traffic figures are for the f32 cache
    tinfo = json.load(open(tpath)) if os.path.exists(tpath) and kv == myos.KV_F32 else {}
    if path_name in ("persistent", "streamed"):
        launch_bytes = b_tok * args.decode
        launch_s = dd / args.steps * 1e-3
        achieved = launch_bytes / launch_s
        traffic, tsrc = committed_traffic(is7b, path_name, args.prompt, args.decode, args.kv)
        roofline = {"bound": "hbm",
                    "kernel": f"{'decode_persistent_kernel' if path_name == 'persistent' else 'decode_wide_kernel'} "
                              f"(one launch: {args.decode} greedy decode steps)",
                    "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4), "traffic": traffic,
                    "traffic_source": tsrc and f"{tsrc}: rocprofv3 --pmc FETCH_SIZE and "
                                               f"WRITE_SIZE of the same launch, scaled by a "
                                               f"copy-kernel calibration (not measured in "
                                               f"this run)",
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
                    "traffic_source": tinfo.get("source"),
                    "algorithmic_bytes": dom["bytes"]}
    m.close()

    pf_long = None if args.no_prefill_2048 else prefill_leg(path, shape, kv, 2048)
    if pf_long:
        log(f"prefill 2048 ids: {pf_long['device_ms']} ms ({pf_long['tok_s']} tok/s, "
            f"{pf_long['mfma_frac_alg']} of the bf16 MFMA peak counted algorithmically)")

    legs = {}
    if other_legs(args, is7b):
        todo = []
        if not args.no_long_context:
            todo.append(("long_context", path, shape, myos.KV_BF16, 2048, 256, False))
        if not args.no_7b:
            todo.append(("qwen25_7b_s1", PATH_7B, myos.preset(myos.SHAPE_QWEN25_7B), myos.KV_F32,
                         128, 128, True))
        for name, lpath, lshape, lkv, n_p, n_d, l7b in todo:
            # a leg that cannot run (its weights file missing, say) reports why; the
            # headline line still prints
            try:
                v = decode_leg(lpath, lshape, lkv, n_p, n_d, l7b)
                log(f"{name}: {v['decode_tok_s']} tok/s ({v['decode_roofline']['frac']} of the HBM "
                    f"roofline), device ms {v['device_ms']}, {v['decode_path']} path")
            except Exception as e:
                v = {"error": str(e)[-300:]}
                log(f"{name}: not measured ({v['error']})")
            legs[name] = v

    micro = None if args.no_gemv_microbench else gemv_microbench()
    if micro:
        log("gemv microbench: " + ", ".join(f"{n} {v['avg_us']}us {v['GBps']}GB/s"
                                             for n, v in micro.items()))

    cpu = None
    if cpu_res:
        cores = host_cores()
        r = cpu_res[cores]
        cpu = {"value": round(n_cpu / r["decode_s"], 3), "unit": "tok/s", "cores": cores,
               "kind": "port",
               "sample": f"same weights file and {args.prompt} prompt ids: prefill then {n_cpu} "
                         f"greedy decode steps on the C oracle (AVX2 32-row GEMV over a "
                         f"row-span thread pool), median of {args.cpu_repeats} runs after a "
                         f"warm-up, at {cores} threads (host nproc {host_nproc()}; the benchmark "
                         f"hosts allot 16 cores per GPU) and at 8 threads",
               "host_nproc": host_nproc(),
               "prefill_tok_s": round(len(prompt) / r["prefill_s"], 2),
               "threads8_decode_tok_s": round(n_cpu / cpu_res[8]["decode_s"], 3) if 8 in cpu_res else None,
               "threads8_prefill_tok_s": round(len(prompt) / cpu_res[8]["prefill_s"], 2) if 8 in cpu_res else None}

    line = {
        "metric": METRIC, "value": round(decode_tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None if is7b else round(decode_tok_s / REF_CPU_DECODE_TOK_S, 2),
        "dtype": "bf16", "data": "synthetic: random-init N(0,0.02) bf16 weights (seed 0), "
                                 "uniform prompt ids (seed 2024)",
        "config": {"workload": workload_name(is7b, args.prompt, args.decode, args.kv),
                   "prompt_ids": args.prompt, "decode_steps": args.decode, "batch": 1,
                   "max_seq": max_seq, "kv_cache": args.kv,
                   "accumulate": "f32 accumulate over bf16 weights; activations enter the "
                                 "products split into bf16 hi + lo terms (16 significant bits) "
                                 "in the MFMA prefill" + (
                                     " and in the register-resident decode kernel's gate/up, "
                                     "down and head (v_dot2); its QKV, o and attention keep f32 "
                                     "activations" if path_name == "persistent" else
                                     "; the decode path keeps f32 activations"),
                   "decode_path": path_name, "graph": not args.no_graph,
                   "parallelism": "single GPU"},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "decode_ms_per_token": round(td / (args.steps * args.decode) * 1e3, 4),
        "device_ms": {"prefill": round(dp / args.steps, 3), "decode": round(dd / args.steps, 3)},
        "decode_roofline": {"bytes_per_token": int(b_tok), "achieved_GBps":
                            round(decode_tok_s * b_tok / 1e9, 1), "peak_GBps": HBM_PEAK / 1e9,
                            "frac": round(decode_frac, 4)},
        "prefill_roofline": pf_roof,
        "roofline": roofline, "parity": parity, "arena": arena,
        "per_kernel_path": kernels, "prefill_2048": pf_long, "other_workloads": legs or None,
        "gemv_microbench": micro,
        "t_load_s": round(t_load, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
