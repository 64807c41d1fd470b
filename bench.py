#!/usr/bin/env python3
"""Batch-1 greedy decode throughput on one MI355X.

Workload (default): the Mistral-7B-shape model -- dim 4096, 32 layers, 32
heads (head_dim 128), 8 KV heads, FFN 14336, vocab 32000, RoPE theta 1e6 --
with seeded N(0, 0.02) weights quantized to Q4_0 (output.weight Q6_K), KV
cache sized to 4096 positions, a random 32-token prompt and then greedy
decode steps.  A step is one token's whole forward (embedding lookup, 32
layers, output projection, argmax) replayed as one hipGraph with the token,
position, weights and KV already resident in HBM.

Prints one JSON line.  `value` is decode tokens/s over exactly --steps timed
steps.  `roofline` is the dominant kernel (the fused rmsnorm + gate/up +
SwiGLU matvec) timed with HIP events on its stream; `token_roofline` is the
whole step against the weights + KV byte floor.  `cpu_baseline` is the
oracle (a C restatement of the reference's CPU forward) on a bounded sample
of the same workload, whose greedy tokens are also compared with the GPU's.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode tok/s batch-1 @7B-shape Q4_0; matvec HBM GB/s vs ~8 TB/s peak"
HBM_PEAK_GBS = 8000.0


def host_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode steps (tokens)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode steps before timing")
    ap.add_argument("--cpu-tokens", type=int, default=8, help="decode tokens in the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the decode path runs on a single MI355X).", file=sys.stderr)
        return 2

    import numpy as np

    import talos_amd as T
    from talos_amd import configs

    wl = configs.mistral7b_q4(ctx=4096)
    spec = wl.spec
    P = wl.prompt_len
    if P + max(args.steps, args.warmup) > spec.context_length:
        print(f"--steps/--warmup exceed the KV capacity ({spec.context_length - P})", file=sys.stderr)
        return 2
    nthreads = host_threads()
    log(f"generating {wl.name} (seed {spec.seed}) with {nthreads} threads")
    t = time.perf_counter()
    model = T.Model.synth(spec, nthreads=nthreads)
    log(f"  generated in {time.perf_counter() - t:.1f}s; uploading + first graph")
    prompt = [int(x) for x in np.random.default_rng(spec.seed + 1).integers(0, spec.vocab_size, P)]

    def prefill() -> int:
        model.reset()
        am = 0
        for p, tok in enumerate(prompt):
            _, am = model.forward_token(tok, p, want_logits=False)
        return am

    t = time.perf_counter()
    first = prefill()
    log(f"  prefill (incl. upload) {time.perf_counter() - t:.1f}s")
    if args.warmup:
        model.decode_greedy(first, P, args.warmup)
    first = prefill()
    t0 = time.perf_counter()
    toks = model.decode_greedy(first, P, args.steps)  # synchronizes at the end
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    log(f"timed {args.steps} steps: {dt * 1e3:.2f} ms -> {tok_s:.1f} tok/s")

    # Dominant kernel, timed with HIP events on the stream it runs on.
    us, kbytes = model.bench_kernel("gateup", 256)
    k_gbs = kbytes / (us * 1e-6) / 1e9
    per_kernel = {}
    for kind in ("qkv", "oproj", "gateup", "down", "output"):
        kus, kb = model.bench_kernel(kind, 64)
        per_kernel[kind] = {"us": round(kus, 2), "GB/s": round(kb / (kus * 1e-6) / 1e9, 1),
                            "bytes": int(kb)}
    log(f"per-kernel: {per_kernel}")

    # Whole-step floor: all weights once + KV read (mean seq) + KV write.
    wbytes = configs.bytes_per_token_weights(spec)
    kvpos = configs.kv_bytes_per_position(spec)
    mean_seq = P + (args.steps + 1) / 2.0
    tok_bytes = wbytes + kvpos * mean_seq + kvpos
    tok_gbs = tok_bytes * tok_s / 1e9

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        log(f"CPU baseline: oracle with {nthreads} threads, {P}-token prompt + {args.cpu_tokens} decode tokens")
        ref = O.OracleModel(model.gguf_view(), nthreads=nthreads)
        tok = None
        for p, t_ in enumerate(prompt):
            lg = ref.forward(t_, p)
        tok = O.argmax(lg)
        cpu_toks = []
        c0 = time.perf_counter()
        for i in range(args.cpu_tokens):
            cpu_toks.append(tok)
            lg = ref.forward(tok, P + i)
            tok = O.argmax(lg)
        cdt = time.perf_counter() - c0
        gpu_seq = [int(first)] + [int(x) for x in toks[: args.cpu_tokens - 1]]
        match = cpu_toks == gpu_seq
        log(f"  cpu {args.cpu_tokens / cdt:.2f} tok/s; greedy tokens match GPU: {match}")
        ref.close()
        cpu = {"value": round(args.cpu_tokens / cdt, 3), "unit": "tok/s", "cores": nthreads,
               "kind": "port",
               "sample": f"C restatement of the reference CPU forward (oracle/talos_oracle.c), "
                         f"same model and {P}-token prompt, {args.cpu_tokens} greedy decode tokens "
                         f"(prefill untimed); greedy tokens identical to the GPU run: {match}"}

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "mistral7b_q4: dim 4096, 32 layers, 32 heads (hd 128), 8 KV heads, "
                               "FFN 14336, vocab 32000, RoPE 1e6, Q4_0 matrices + Q6_K output, "
                               "random 32-token prompt then greedy decode, KV ctx 4096",
                   "batch": 1, "prompt_tokens": P, "weights": "Q4_0/Q6_K", "kv": "f32"},
        "roofline": {"bound": "hbm", "kernel": "k_gateup (rmsnorm + gate/up Q4_0 matvec + SwiGLU)",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": int(kbytes), "us_per_launch": round(us, 3)},
        "token_roofline": {"bytes_per_token": int(tok_bytes), "achieved": round(tok_gbs, 1),
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(tok_gbs / HBM_PEAK_GBS, 4),
                           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / tok_bytes, 1)},
        "per_kernel": per_kernel,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    model.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
