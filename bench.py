#!/usr/bin/env python3
"""Batch-1 greedy decode throughput on one MI355X.

Workload (default): the Mistral-7B-shape model -- dim 4096, 32 layers, 32
heads (head_dim 128), 8 KV heads, FFN 14336, vocab 32000, RoPE theta 1e6 --
with seeded N(0, 0.02) weights quantized to Q4_0 (output.weight Q6_K), KV
cache sized to 4096 positions, a random 32-token prompt and then greedy
decode steps.  A step is one token's whole forward (embedding lookup, 32
layers, output projection, argmax), which runs as one persistent kernel
launch with the token, position, weights and KV already resident in HBM.

Prints one JSON line.  `value` is decode tokens/s over exactly --steps timed
steps.  `roofline` is that kernel (the whole decode step) timed with HIP
events on its stream at the middle position of the timed run: algorithmic
bytes per step (weights once, K/V read and written, logits) over the mean
step time.  `cpu_baseline` is the oracle (a C restatement of the
reference's CPU forward) on a bounded sample of the same model, whose greedy
tokens are also compared with the GPU's.

The default run also reports, after the headline line's own measurements,
`small_models` (tok/s of the tiny F32 and GQA Q8_0 models) and `lc` (the
long-context case below: its prompt tok/s, decode tok/s and roofline);
--no-extra skips them.  `parity` records the GPU/CPU comparison
of the CPU baseline's sample (greedy tokens and worst max-abs logit
difference); a failed comparison makes the run exit with status 3.

--workload lc: the long-context case -- the same 7B shape with every matrix
in Q8_0, the KV cache filled to 16384 positions by a device prompt feed of
a uniform random 16384-token prefix (talos_hip_prefill; --lc-fill kv writes
a seeded K/V state instead), then 64 greedy decode steps at positions
16384..16447.  Its CPU baseline runs the oracle from the GPU's cache.
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
PHASES = ["qkv_work", "attn_barrier", "attn_work", "o_barrier", "o_stage", "o_work", "gateup_barrier",
          "gateup_stage", "gateup_work", "down_barrier", "down_stage", "down_work", "next_barrier", "next_stage"]


def host_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


TRAFFIC_FILE = os.path.join("profiles", "k_mega_7b_q4_pmc_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the decode step, from the rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE runs summarized in TRAFFIC_FILE (scaled by a copy
    kernel of known size), or None."""
    try:
        with open(os.path.join(ROOT, TRAFFIC_FILE)) as f:
            for line in f:
                if line.startswith("TRAFFIC_BYTES_PER_LAUNCH"):
                    return int(line.split("=")[1])
    except (OSError, ValueError):
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def phase_breakdown(tl, n_layer: int, per_layer: int = 20, bar: int = 16) -> dict:
    """Mean microseconds per layer of each phase of one step, from the
    latest workgroup's mark at each phase boundary (marks per layer: 0 qkv
    staged, 1 qkv end, 2 attention barrier passed, 3 attention end, 4 o
    staged, 5 o end, 6 gate/up staged, 7 gate/up end, 8 down staged, 9 down
    end; bar + 0..3: barrier passed before the qkv, o, gate/up and down
    staging)."""
    import numpy as np
    mx = tl.max(axis=0)
    seg = {k: [] for k in PHASES}
    for l in range(n_layer):
        b = l * per_layer
        m = lambda i: mx[b + i]
        vals = [m(1) - m(0), m(2) - m(1), m(3) - m(2), m(bar + 1) - m(3), m(4) - m(bar + 1), m(5) - m(4),
                m(bar + 2) - m(5), m(6) - m(bar + 2), m(7) - m(6), m(bar + 3) - m(7), m(8) - m(bar + 3),
                m(9) - m(8)]
        for k, v in zip(PHASES[:12], vals):
            seg[k].append(v)
        if l + 1 < n_layer:
            seg["next_barrier"].append(mx[b + per_layer + bar] - m(9))
            seg["next_stage"].append(mx[b + per_layer] - mx[b + per_layer + bar])
    return {k: round(float(np.mean(v)) / 1e3, 2) for k, v in seg.items() if v}


def matvec_microbench(T) -> dict:
    """W[4096 x 4096] . x[4096] in F32, Q8_0 and Q4_0 (W ~ N(0, 0.02)),
    rotating over enough resident copies (> 256 MB) that every launch
    streams W from HBM.  GB/s of algorithmic bytes (W + x + y) per launch,
    launched back to back on one stream.  `copy_us` is a plain device copy
    of the matrix's size launched the same way: one launch of a kernel that
    reads those bytes (and writes as many) costs at least that, so
    `copy_frac` (the matvec's bytes over copy_us, against peak) is what a
    single-launch matvec of this size can reach."""
    n = 4096
    be = T.HipBackend(1, 32, 8, n, n, 32, 16)
    w = T.synth_normal(7, "matvec.W", 0, n * n, 0.02)
    res = {}
    for name, t, data in (("F32", T.GGML_F32, w), ("Q8_0", T.GGML_Q8_0, T.quantize(T.GGML_Q8_0, w)),
                          ("Q4_0", T.GGML_Q4_0, T.quantize(T.GGML_Q4_0, w))):
        copies = max(2, (512 << 20) // data.nbytes + 1)
        names = [f"mv.{name}.{i}" for i in range(copies)]
        for nm in names:
            be.upload(nm, data, t, n, n)
        us, b = be.bench_matvec(names, 256)
        cus = be.bench_copy((data.nbytes + 15) // 16 * 16, 256)
        res[name] = {"us": round(us, 2), "GB/s": round(b / (us * 1e-6) / 1e9, 1),
                     "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes": int(b),
                     "copy_us": round(cus, 2), "copy_frac": round(b / (cus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    be.close()
    log(f"matvec 4096x4096: {res}")
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=("decode", "lc"), default="decode",
                    help="decode: 7B Q4_0 at KV ctx 4096 (default); lc: 7B Q8_0 after a 16384-token prefix")
    ap.add_argument("--lc-fill", choices=("prefill", "kv"), default="prefill",
                    help="lc: fill the 16384-position cache by the device prompt feed or a seeded K/V write")
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (tokens; 128, lc 64)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode steps before timing")
    ap.add_argument("--cpu-prompt", type=int, default=8, help="prompt tokens of the CPU baseline sample")
    ap.add_argument("--cpu-tokens", type=int, default=32, help="greedy decode tokens of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the small-model and long-context sub-objects of the default run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the decode path runs on a single MI355X).", file=sys.stderr)
        return 2

    if args.workload == "lc":
        return run_lc(args)
    if args.steps is None:
        args.steps = 128

    import numpy as np

    import talos_amd as T
    from talos_amd import configs

    wl = configs.mistral7b_q4(ctx=4096)
    spec = wl.spec
    P = wl.prompt_len
    if P + args.warmup + args.steps > spec.context_length:
        print(f"--steps/--warmup exceed the KV capacity ({spec.context_length - P})", file=sys.stderr)
        return 2
    nthreads = host_threads()
    log(f"generating {wl.name} (seed {spec.seed}) with {nthreads} threads")
    t = time.perf_counter()
    model = T.Model.synth(spec, nthreads=nthreads)
    log(f"  generated in {time.perf_counter() - t:.1f}s")
    prompt = [int(x) for x in np.random.default_rng(spec.seed + 1).integers(0, spec.vocab_size, P)]

    def prefill() -> int:
        model.reset()
        am = 0
        for p, tok in enumerate(prompt):
            _, am = model.forward_token(tok, p, want_logits=False)
        return am

    t = time.perf_counter()
    first = prefill()
    log(f"  prefill (incl. weight upload) {time.perf_counter() - t:.1f}s")
    if args.warmup:
        model.decode_greedy(first, P, args.warmup)
    first = prefill()
    t0 = time.perf_counter()
    toks = model.decode_greedy(first, P, args.steps)  # synchronizes at the end
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    log(f"timed {args.steps} steps: {dt * 1e3:.2f} ms -> {tok_s:.1f} tok/s")

    # The decode step is one kernel launch: time it with HIP events on its
    # stream at the middle position of the timed run (K/V rows up to there
    # were written by the run above).
    mid = P + args.steps // 2
    us, sbytes = model.bench_token(int(toks[args.steps // 2 - 1]), mid, 32)
    k_gbs = sbytes / (us * 1e-6) / 1e9
    log(f"decode step at pos {mid}: {us:.1f} us, {sbytes / 1e6:.1f} MB -> {k_gbs:.0f} GB/s")
    copy_bytes = 1 << 30
    cus = model.bench_copy(copy_bytes, 10)
    copy_gbs = 2 * copy_bytes / (cus * 1e-6) / 1e9
    log(f"device copy of 1 GiB: {cus:.1f} us -> {copy_gbs:.0f} GB/s (read + write)")
    # per-phase marks exist only in the persistent kernel
    phases = (phase_breakdown(model.phase_timeline(int(toks[args.steps // 2 - 1]), mid), spec.n_layer)
              if model.path() == "persistent" else None)
    log(f"phase us per layer: {phases}")

    # The host-buffer boundary (talos_hip_forward: embedding row in, logits
    # out over PCIe), for comparison with the device-resident token loop.
    model.reset()
    for p, tok in enumerate(prompt):
        model.forward_token(tok, p, want_logits=False)
    t1 = time.perf_counter()
    npc = min(32, args.steps)
    for i in range(npc):
        lg = model.forward_gpu(int(toks[i]), P + i)
    pcie_tok_s = npc / (time.perf_counter() - t1)
    log(f"host-boundary forward (x_embed H2D + logits D2H): {pcie_tok_s:.1f} tok/s")

    matvec = matvec_microbench(T)

    # Whole-run floor: all weights once + KV read (mean seq) + KV write.
    wbytes = configs.bytes_per_token_weights(spec)
    kvpos = configs.kv_bytes_per_position(spec)
    mean_seq = P + (args.steps + 1) / 2.0
    tok_bytes = wbytes + kvpos * mean_seq + kvpos
    tok_gbs = tok_bytes * tok_s / 1e9

    cpu = None
    parity = None
    if not args.no_cpu and args.cpu_tokens > 0:
        from oracle import oracle as O
        simd = O.host_has_avx2()
        n_fw = args.cpu_prompt + args.cpu_tokens
        log(f"CPU baseline: oracle ({'-O3 -mavx2' if simd else 'parity'} build) with {nthreads} threads, "
            f"{args.cpu_prompt}-token prompt + {args.cpu_tokens} greedy tokens ({n_fw} forwards)")
        ref = O.OracleModel(model.gguf_view(), nthreads=nthreads, simd=simd)
        c0 = time.perf_counter()
        cpu_logits = []
        for p, t_ in enumerate(prompt[: args.cpu_prompt]):
            lg = ref.forward(t_, p)
            cpu_logits.append(lg)
        tok = O.argmax(lg)
        cpu_toks = []
        for i in range(args.cpu_tokens):
            cpu_toks.append(tok)
            lg = ref.forward(tok, args.cpu_prompt + i)
            cpu_logits.append(lg)
            tok = O.argmax(lg)
        cdt = time.perf_counter() - c0
        ref.close()
        # the same sequence on the GPU, logits compared at every step
        model.reset()
        worst, gpu_toks = 0.0, []
        seq = prompt[: args.cpu_prompt] + cpu_toks
        for p, t_ in enumerate(seq):
            lg, am = model.forward_token(t_, p)
            worst = max(worst, float(np.abs(lg - cpu_logits[p]).max()))
            if p >= args.cpu_prompt - 1:
                gpu_toks.append(int(am))
        match = gpu_toks[: len(cpu_toks)] == cpu_toks
        log(f"  cpu {n_fw / cdt:.3f} tok/s over {cdt:.1f}s; greedy tokens match GPU: {match}, "
            f"worst max-abs logit diff {worst:.3e}")
        parity = {"greedy_match": match, "worst_max_abs_logit": worst, "tol": 1e-3, "forwards": n_fw}
        cpu = {"value": round(n_fw / cdt, 4), "unit": "tok/s", "cores": nthreads, "kind": "port",
               "sample": f"oracle/talos_oracle.c ({'-O3 -mavx2 build, bit-identical to the parity build' if simd else 'parity build'}; "
                         f"a C restatement of the reference CPU forward, {nthreads} OpenMP threads) on the same "
                         f"model: {args.cpu_prompt}-token prompt + {args.cpu_tokens} greedy tokens = {n_fw} "
                         f"forwards, all timed.  The CPU step is weight-bound (4.03 GB of weights against at most "
                         f"42 MB of K/V at position 160), so this rate holds for the full 32 + 128 workload "
                         f"within about 1%"}

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
        "path": model.path(),
        "config": {"workload": "mistral7b_q4: dim 4096, 32 layers, 32 heads (hd 128), 8 KV heads, "
                               "FFN 14336, vocab 32000, RoPE 1e6, Q4_0 matrices + Q6_K output, "
                               "random 32-token prompt then greedy decode, KV ctx 4096",
                   "batch": 1, "prompt_tokens": P, "weights": "Q4_0/Q6_K", "kv": "f32"},
        "roofline": {"bound": "hbm", "kernel": "k_mega (persistent decode step: 32 layers + output + argmax)",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": f"rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE ({TRAFFIC_FILE})",
                     "bytes_per_launch": int(sbytes), "us_per_launch": round(us, 2), "pos": mid,
                     "copy_kernel_GBs": round(copy_gbs, 1)},
        "token_roofline": {"bytes_per_token": int(tok_bytes), "achieved": round(tok_gbs, 1),
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(tok_gbs / HBM_PEAK_GBS, 4),
                           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / tok_bytes, 1)},
        "phase_us_per_layer": phases,
        "host_boundary_tok_s": round(pcie_tok_s, 2),
        "matvec_4096x4096": matvec,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    model.close()
    if not args.no_extra:
        out["small_models"] = small_models()
        out["lc"] = lc_measure(args)
    print(json.dumps(out), flush=True)
    if parity is not None and not (parity["greedy_match"] and parity["worst_max_abs_logit"] <= parity["tol"]):
        log("GPU/CPU parity check FAILED: the measurement is invalid")
        return 3
    return 0


def small_models() -> dict:
    """tok/s of the tiny F32 (8 + 64 greedy steps) and GQA Q8_0 (16 + 256)
    models: whole runs on the device, prompt fed then the greedy loop."""
    import numpy as np

    import talos_amd as T
    from talos_amd import configs
    res = {}
    for wl in (configs.tiny_f32(), configs.gqa_q8()):
        m = T.Model.synth(wl.spec)
        prompt = np.random.default_rng(wl.spec.seed + 1).integers(0, wl.spec.vocab_size, wl.prompt_len)
        _, first = m.prefill(prompt, 0, want_logits=False)  # uploads, warms
        m.decode_greedy(first, wl.prompt_len, 8)
        m.reset()
        t0 = time.perf_counter()
        _, first = m.prefill(prompt, 0, want_logits=False)
        t1 = time.perf_counter()
        m.decode_greedy(first, wl.prompt_len, wl.decode_steps)
        t2 = time.perf_counter()
        res[wl.name] = {"decode_tok_s": round(wl.decode_steps / (t2 - t1), 1),
                        "prompt_tok_s": round(wl.prompt_len / (t1 - t0), 1),
                        "steps": wl.decode_steps, "prompt_tokens": wl.prompt_len, "path": m.path()}
        m.close()
    log(f"small models: {res}")
    return res


def lc_measure(args) -> dict:
    """The long-context case beside the headline one: the 7B shape in Q8_0,
    its cache filled to 16384 positions by talos_hip_prefill of a uniform
    random prefix (timed: prompt tok/s), then 64 greedy steps (decode tok/s
    and the step's roofline at the middle position).  Its parity is the GPU
    tests' (tests/test_gpu_long.py, tests/test_gpu_prefill.py)."""
    import numpy as np

    import talos_amd as T
    from talos_amd import configs
    wl = configs.mistral7b_q8_long()
    spec, P, steps = wl.spec, wl.prompt_len, wl.decode_steps
    nthreads = host_threads()
    t = time.perf_counter()
    model = T.Model.synth(spec, nthreads=nthreads)
    rng = np.random.default_rng(spec.seed + 1)
    prefix = rng.integers(0, spec.vocab_size, P).astype(np.uint32)
    model.prefill(prefix[:64], 0, want_logits=False)  # uploads the weights, sizes the batch buffers
    log(f"lc: model ready in {time.perf_counter() - t:.1f}s")
    t = time.perf_counter()
    _, first = model.prefill(prefix, 0, want_logits=False)
    prefill_s = time.perf_counter() - t
    gemm_f, attn_f = configs.prefill_flops(spec, P)
    log(f"lc: prefill of {P} positions {prefill_s:.2f}s ({P / prefill_s:.0f} tok/s, "
        f"{(gemm_f + attn_f) / prefill_s / 1e12:.0f} TFLOP/s)")
    model.decode_greedy(first, P, 8)
    t0 = time.perf_counter()
    toks = model.decode_greedy(first, P, steps)
    dt = time.perf_counter() - t0
    mid = P + steps // 2
    us, sbytes = model.bench_token(int(toks[steps // 2 - 1]), mid, 16)
    k_gbs = sbytes / (us * 1e-6) / 1e9
    wbytes = configs.bytes_per_token_weights(spec)
    kvpos = configs.kv_bytes_per_position(spec)
    tok_bytes = wbytes + kvpos * (P + (steps + 1) / 2.0) + kvpos
    model.close()
    res = {"workload": f"mistral7b_q8_long: 7B shape, Q8_0 matrices, {P}-token uniform random prompt "
                       f"(talos_hip_prefill), {steps} greedy steps", "tok_s": round(steps / dt, 2), "steps": steps,
           "prefill_tok_s": round(P / prefill_s, 1),
           "prefill": {"seconds": round(prefill_s, 3), "projection_flops": gemm_f, "attention_flops": attn_f,
                       "achieved_tflops": round((gemm_f + attn_f) / prefill_s / 1e12, 1),
                       "note": "projections on f16 matrix cores with x split into hi + lo halves (two "
                               "MFMAs per product), reading tile-contiguous copies of the layer matrices "
                               "(made by the warm-up prefill), attention on f16 matrix cores with q, K, V "
                               "and the probabilities split (three MFMAs per product); f16 MFMA peak "
                               "2500 TFLOP/s"},
           "roofline": {"bound": "hbm", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(k_gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": int(sbytes),
                        "us_per_launch": round(us, 2), "pos": mid},
           "token_roofline_frac": round(tok_bytes * steps / dt / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"lc: {res['tok_s']} tok/s, step at pos {mid}: {us:.1f} us -> {k_gbs:.0f} GB/s")
    return res


LC_TRAFFIC_FILE = os.path.join("profiles", "k_mega_7b_q8_16k_pmc_traffic.md")


def run_lc(args) -> int:
    """Long-context decode: 7B shape, Q8_0, 16384 cached positions, then
    --steps (64) greedy steps."""
    import numpy as np

    import talos_amd as T
    from talos_amd import configs

    wl = configs.mistral7b_q8_long()
    spec = wl.spec
    P = wl.prompt_len
    steps = wl.decode_steps if args.steps is None else args.steps
    if steps < 2 or P + max(steps, args.warmup) > spec.context_length:
        print(f"--steps/--warmup must be in [2, {spec.context_length - P}]", file=sys.stderr)
        return 2
    nthreads = host_threads()
    log(f"generating {wl.name} (seed {spec.seed}) with {nthreads} threads")
    t = time.perf_counter()
    model = T.Model.synth(spec, nthreads=nthreads)
    log(f"  generated in {time.perf_counter() - t:.1f}s")
    rng = np.random.default_rng(spec.seed + 1)
    prefix = rng.integers(0, spec.vocab_size, P).astype(np.uint32)
    t = time.perf_counter()
    model.forward_token(int(prefix[0]), 0, want_logits=False)  # uploads the weights
    log(f"  weight upload + first step {time.perf_counter() - t:.1f}s")
    prefill_tok_s = None
    if args.lc_fill == "prefill":
        chunk = 2048
        t = time.perf_counter()
        for i in range(0, P, chunk):
            _, first = model.prefill(prefix[i:i + chunk], i, want_logits=False)
            log(f"  prefill {min(i + chunk, P)}/{P} positions, {time.perf_counter() - t:.1f}s")
        prefill_tok_s = P / (time.perf_counter() - t)
        fill = f"talos_hip_prefill of a uniform random {P}-token prefix ({prefill_tok_s:.1f} tok/s)"
    else:
        k = rng.standard_normal((spec.n_layer, P, spec.kv_dim), dtype=np.float32) * np.float32(1.28)
        v = rng.standard_normal((spec.n_layer, P, spec.kv_dim), dtype=np.float32) * np.float32(1.28)
        model.kv_write(k, v)
        del k, v
        first = int(prefix[-1])
        fill = f"seeded N(0, 1.28^2) K/V state of {P} positions written to the cache"
    log(f"cache filled: {fill}")
    if args.warmup:
        model.decode_greedy(first, P, args.warmup)
    t0 = time.perf_counter()
    toks = model.decode_greedy(first, P, steps)
    dt = time.perf_counter() - t0
    tok_s = steps / dt
    log(f"timed {steps} steps from pos {P}: {dt * 1e3:.2f} ms -> {tok_s:.1f} tok/s")
    mid = P + steps // 2
    us, sbytes = model.bench_token(int(toks[steps // 2 - 1]), mid, 16)
    k_gbs = sbytes / (us * 1e-6) / 1e9
    log(f"decode step at pos {mid}: {us:.1f} us, {sbytes / 1e6:.1f} MB -> {k_gbs:.0f} GB/s")
    phases = (phase_breakdown(model.phase_timeline(int(toks[steps // 2 - 1]), mid), spec.n_layer)
              if model.path() == "persistent" else None)
    log(f"phase us per layer: {phases}")
    wbytes = configs.bytes_per_token_weights(spec)
    kvpos = configs.kv_bytes_per_position(spec)
    tok_bytes = wbytes + kvpos * (P + (steps + 1) / 2.0) + kvpos
    tok_gbs = tok_bytes * tok_s / 1e9

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        # Restore the cache to the prefix (the timed run wrote P..P+steps-1,
        # which the oracle recomputes) and run two greedy steps from it.
        log(f"CPU baseline: oracle with {nthreads} threads from the GPU's {P}-position cache, 2 decode steps")
        k, v = model.kv_read(P)
        ref = O.OracleModel(model.gguf_view(), nthreads=nthreads)
        ref.set_kv(k, v)
        del k, v
        c0 = time.perf_counter()
        tok, cpu_toks = first, []
        for i in range(2):
            tok = O.argmax(ref.forward(tok, P + i))
            cpu_toks.append(tok)
        cdt = time.perf_counter() - c0
        ref.close()
        match = cpu_toks == [int(x) for x in toks[:2]]
        log(f"  cpu {2 / cdt:.4f} tok/s over {cdt:.1f}s; greedy tokens match GPU: {match}")
        cpu = {"value": round(2 / cdt, 5), "unit": "tok/s", "cores": nthreads, "kind": "port",
               "sample": f"oracle/talos_oracle.c ({nthreads} OpenMP threads; attention is the reference's "
                         f"serial loop) on the same model: 2 greedy decode steps at pos {P}, {P + 1} from "
                         f"the GPU's {P}-position cache; greedy tokens identical to the GPU: {match}"}

    traffic = None
    try:
        with open(os.path.join(ROOT, LC_TRAFFIC_FILE)) as f:
            for line in f:
                if line.startswith("TRAFFIC_BYTES_PER_LAUNCH"):
                    traffic = int(line.split("=")[1])
    except (OSError, ValueError):
        pass
    out = {
        "metric": "decode tok/s batch-1 @7B-shape Q8_0 after a 16384-token prefix (long context)",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"mistral7b_q8_long: 7B shape, Q8_0 matrices (output and embedding too), "
                               f"KV filled to {P} positions ({fill}), then {steps} greedy steps, "
                               f"KV capacity {spec.context_length}",
                   "batch": 1, "prefix_tokens": P, "weights": "Q8_0", "kv": "f32"},
        "roofline": {"bound": "hbm", "kernel": "k_mega (persistent decode step: 32 layers + output + argmax)",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": f"rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE ({LC_TRAFFIC_FILE})",
                     "bytes_per_launch": int(sbytes), "us_per_launch": round(us, 2), "pos": mid},
        "token_roofline": {"bytes_per_token": int(tok_bytes), "achieved": round(tok_gbs, 1),
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(tok_gbs / HBM_PEAK_GBS, 4),
                           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / tok_bytes, 1)},
        "phase_us_per_layer": phases,
        "prefill_tok_s": None if prefill_tok_s is None else round(prefill_tok_s, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    model.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
