#!/usr/bin/env python3
"""Gemma-2B Int8Blocks decode throughput on one MI355X, with the other
benchmark configurations measured beside it.

Headline workload (the `value` of the JSON line): the full Gemma-2B shape (18
layers, width 2048, 8 query heads / 1 KV head of 256, FFN 16384, vocabulary
256000 with the tied embedding), seeded N(0, 0.02) weights (norms N(0, 0.1))
quantized to Int8Blocks, a 512-token seeded uniform prompt, greedy decode with
an fp16 KV cache.  A step is one decode token: embed, 18 layers, final norm,
the tied lm_head over 256000 rows and the on-device argmax that feeds the next
step.  The prefill is untimed; W warmup decode steps run in a separate
sequence; then exactly K decode steps are timed after a fresh 512-token
prefill, bracketed by device synchronisation.

Beside it, on the same weights (the `configs` object):
  prefill       the 2048-token prompt as one step (every linear an int8 MFMA
                GEMM of M = 2048): ms, tok/s, int8 TOP/s and its fraction of
                the MFMA peak;
  long_context  an 8064-token prompt, then decode to the end of the
                8192-position window (128 tokens): tok/s and HBM fraction;
  lockstep      16 sequences of 1024-token prompts decoding 128 tokens in
                lockstep: aggregate tok/s and HBM fraction;
and the CPU baseline: the oracle's C decoder on the host cores, config 2
decode after its 512-token prefill and the two-layer workload end to end.

Prints one JSON line on stdout (everything else goes to stderr).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
# HBM bytes a launch of the dominant decode kernels moves, from two rocprofv3
# counter passes over the current kernels (FETCH_SIZE scaled by what it reads
# for a 256 MiB copy, plus WRITE_SIZE); the passes, their commands and the
# calibration are in TRAFFIC_SOURCE.
TRAFFIC_SOURCE = "profiles/decode_kernels_gemma2b_hbm_traffic.md"
MEASURED_TRAFFIC = {"gate_up": 71542751, "lm_head": 558436311, "down": 35961103}
METRIC = "Gemma-2B Q8_0 decode tok/s (b=1, ctx 512) + % of HBM roofline"
STAGE_LABELS = {
    "gate_up": "gateup_geglu_kernel (post-attention norm + gate|up 2048 -> 2x16384 + GeGLU + Q8)",
    "lm_head": "lmhead_argmax_kernel (tied lm_head 2048 -> 256000 + first-maximum fold)",
    "down": "q8_matvec_kernel<4,4,2> (down 16384 -> 2048 + residual)",
}
DATA = ("synthetic: seeded N(0,0.02) weights / N(0,0.1) norms quantized to Int8Blocks, "
        "seeded uniform prompt ids")
ORACLE_BUILD = ("gcc -O3 -fopenmp -ffp-contract=off -march=x86-64-v2, the int8 block dot and "
                "the fp32 row dot built for AVX-512F / AVX2 / baseline and picked at load time")


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def host_cpu() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def stage_bytes(shape, stage: str) -> int:
    """Algorithmic HBM bytes of one launch of a one-token product kernel: the
    Int8Blocks weight bytes (17/16 byte per element) plus the activation rows
    it must read and write once."""
    w, f, v = shape.width, shape.intermediate, shape.vocab
    q8 = lambda n: n * 17 // 16  # noqa: E731 -- an Int8Blocks row of n elements
    if stage == "gate_up":  # fp32 residual row + norm weights in, Q8 GeGLU row out
        return q8(2 * f * w) + 2 * w * 4 + q8(f)
    if stage == "lm_head":  # Q8 final-norm row in, fp32 logits out
        return q8(v * w) + q8(w) + v * 4
    if stage == "down":  # Q8 GeGLU row in, fp32 residual read and written
        return q8(f * w) + q8(f) + 2 * w * 4
    raise ValueError(stage)


def linear_ops(shape) -> int:
    """Int8 operations of one row through every linear of the layers."""
    return shape.layers * 2 * (shape.width * (shape.query_width + 2 * shape.kv_width)
                               + shape.query_width * shape.width
                               + 2 * shape.width * shape.intermediate
                               + shape.intermediate * shape.width)


# ---- the headline: config 2 decode ---------------------------------------------------
def headline_decode(args, G, torch, decoder, shape, use_graph):
    prompt = G.prompt_ids(0xC0FFEE + 2, shape.vocab, args.prompt)
    # warmup: its own sequence (graph instantiation, first launches)
    decoder.generate(prompt, args.warmup + 1, eos=-1, use_graph=use_graph)
    # timed: prefill + first token untimed, then exactly K decode steps
    _, stats = decoder.generate(prompt, 1, eos=-1, use_graph=use_graph)
    log(f"prefill of {args.prompt} tokens: {stats.prefill_seconds * 1e3:.1f} ms")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    decoder.decode(args.steps, use_graph=use_graph)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    tok_s = args.steps / seconds
    first_l = args.prompt + 1
    step_bytes = sum(G.algorithmic_decode_bytes(shape, L)
                     for L in range(first_l, first_l + args.steps)) / args.steps
    step_gbs = step_bytes * tok_s / 1e9
    tokens = decoder.tokens(args.prompt, args.steps + 1)
    log(f"decode: {tok_s:.1f} tok/s, {seconds / args.steps * 1e3:.3f} ms/step, "
        f"{step_gbs:.0f} GB/s of {step_bytes / 1e9:.4f} GB/token; first ids {list(tokens[:6])}")

    # the stage breakdown: every launch group of K more steps bracketed by HIP
    # events on the decoder's stream (the event packets add about a
    # microsecond to each bracket)
    decoder.generate(prompt, 1, eos=-1, use_graph=False)
    decoder.set_timing(True)
    decoder.decode(args.steps, use_graph=False)
    timing = decoder.timing()
    decoder.set_timing(False)
    total_ms = sum(ms for ms, _ in timing.values())
    for name, (ms, n) in sorted(timing.items(), key=lambda kv: -kv[1][0]):
        if n:
            log(f"  {name:10s} {ms / args.steps * 1e3:8.1f} us/step  {n // args.steps:3d} launches/step"
                f"  {100 * ms / total_ms:5.1f} %")
    # the dominant product kernel's own duration: launched alone, back to back
    # over every layer's weights (so from HBM, as in a step), between two HIP
    # events on the decoder's stream
    dominant = max(("gate_up", "lm_head", "down"), key=lambda k: timing[k][0])
    ms, launches = decoder.time_kernel(dominant, max(1, args.steps // 8))
    per_launch_s = ms / launches / 1e3
    launch_bytes = stage_bytes(shape, dominant)
    achieved = launch_bytes / per_launch_s / 1e9
    roofline = {"bound": "hbm", "kernel": STAGE_LABELS[dominant], "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": MEASURED_TRAFFIC.get(dominant), "traffic_source": TRAFFIC_SOURCE,
                "bytes_per_launch": launch_bytes, "avg_launch_us": round(per_launch_s * 1e6, 2)}
    return {"tok_s": tok_s, "seconds": seconds, "step_bytes": step_bytes, "step_gbs": step_gbs,
            "roofline": roofline}


# ---- config 3: the 2048-token prefill as one step ----------------------------------------
def prefill_config(args, G, torch, decoder, shape, rows=2048, warmup=1, timed=3):
    prompt = G.prompt_ids(0xC0FFEE + 3, shape.vocab, rows).astype(np.uint32)
    ids = torch.from_numpy(prompt.copy()).to("cuda")
    logits = torch.empty(shape.vocab, dtype=torch.float32, device="cuda")

    def once():
        decoder.begin_sequence()
        decoder.step(ids.data_ptr(), rows, logits.data_ptr(), 1)

    for _ in range(warmup):
        once()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(timed):
        once()
    torch.cuda.synchronize()
    seconds = (time.perf_counter() - t0) / timed
    int_ops = rows * linear_ops(shape) + 2 * shape.width * shape.vocab  # lm_head: the last row
    tops = int_ops / seconds / 1e12
    log(f"config 3 prefill of {rows} tokens: {seconds * 1e3:.2f} ms, {int_ops / 1e12:.3f} T int8 "
        f"ops, {tops:.1f} TOP/s")
    return {"workload": f"Gemma-2B Int8Blocks prefill, {shape.layers} layers, {rows}-token prompt "
                        "as one step, last-row logits",
            "ms": round(seconds * 1e3, 3), "tok_s": round(rows / seconds, 1),
            "int8_tops": round(tops, 2), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
            "peak_tops": INT8_PEAK_TOPS,
            "counted": "2 M K N int8 ops over every linear plus the last row's lm_head; "
                       "attention's fp64 work not counted",
            "steps": timed, "warmup": warmup}


# ---- config 4: decode to the end of the 8192-position window -------------------------------
def long_context_config(args, G, torch, decoder, shape, prompt_len=8064):
    steps = shape.max_positions - prompt_len - 1  # the first id comes from the prefill
    prompt = G.prompt_ids(0xC0FFEE + 4, shape.vocab, prompt_len)
    decoder.generate(prompt, 1, eos=-1, use_graph=True)  # prefill + first id, untimed
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    decoder.decode(steps, use_graph=True)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    tok_s = steps / seconds
    step_bytes = sum(G.algorithmic_decode_bytes(shape, L)
                     for L in range(prompt_len + 1, prompt_len + 1 + steps)) / steps
    gbs = step_bytes * tok_s / 1e9
    log(f"config 4 long context: {tok_s:.1f} tok/s, {seconds / steps * 1e3:.3f} ms/step, "
        f"{gbs:.0f} GB/s of {step_bytes / 1e9:.4f} GB/token")
    return {"workload": f"Gemma-2B Int8Blocks greedy decode, {shape.layers} layers, "
                        f"{prompt_len}-token prompt, {steps} timed decode steps to the end of the "
                        f"{shape.max_positions}-position window",
            "tok_s": round(tok_s, 2), "ms_per_step": round(seconds / steps * 1e3, 4),
            "bytes_per_token": int(step_bytes), "achieved_gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "steps": steps}


# ---- config 5: 16 sequences in lockstep ----------------------------------------------------
def lockstep_config(args, G, torch, decoder, shape, sequences=16, prompt_len=1024, steps=128,
                    warmup=4):
    """Its own decoder: a sequence's cache holds the workload's positions
    (1024 + 128 + the warmup), which is also the span the lockstep attention
    spreads its key splits over."""
    threads = args.threads if args.threads > 0 else (os.cpu_count() or 1)
    shape = G.DecoderShape.gemma_2b(layers=args.layers,
                                    max_positions=prompt_len + steps + warmup + 1,
                                    max_step_rows=prompt_len)
    decoder = G.Decoder(shape)
    decoder.fill_synthetic(threads)
    batch = G.Batch(decoder, sequences)
    prompts = [G.prompt_ids(0xC0FFEE + 5 + 1000 * s, shape.vocab, prompt_len)
               for s in range(sequences)]

    def prefill_all():
        for s, prompt in enumerate(prompts):
            batch.prefill(s, prompt)

    prefill_all()
    batch.decode(warmup, use_graph=True)
    prefill_all()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    batch.decode(steps, use_graph=True)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    batch.close()
    decoder.close()
    tok_s = sequences * steps / seconds
    step_bytes = sum(G.algorithmic_batch_step_bytes(shape, [prompt_len + k + 1] * sequences)
                     for k in range(steps)) / steps
    gbs = step_bytes * steps / seconds / 1e9
    log(f"config 5 lockstep: {tok_s:.1f} tok/s, {seconds / steps * 1e3:.3f} ms/step, {gbs:.0f} GB/s "
        f"of {step_bytes / 1e9:.4f} GB/step")
    return {"workload": f"Gemma-2B Int8Blocks lockstep greedy decode, {shape.layers} layers, "
                        f"{sequences} sequences x ({prompt_len} prompt + {steps} timed steps), "
                        "fp16 KV caches",
            "tok_s": round(tok_s, 1), "ms_per_step": round(seconds / steps * 1e3, 4),
            "bytes_per_step": int(step_bytes), "achieved_gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "sequences": sequences, "steps": steps}


# ---- the CPU baseline -----------------------------------------------------------------------
def cpu_baseline(args, threads: int, decode_bytes) -> dict:
    """The oracle's Q8 decoder (C, OpenMP over the host cores): config 2's
    decode after its 512-token prefill (a bounded sample of decode steps), and
    the two-layer workload (16-token prompt, 32 greedy tokens) end to end;
    beside it the reference's own arithmetic (fp32 activations and KV cache,
    the weights dequantized in the product) on a bounded decode sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    O.lib()
    prompt_tokens = args.prompt
    shape = O.gemma_2b_shape(layers=args.layers, max_positions=prompt_tokens + 1024)
    model = O.Model(shape, O.MODE_Q8)
    t0 = time.perf_counter()
    assert model.fill_synthetic() == 0
    load = time.perf_counter() - t0
    prompt = O.prompt_ids(0xC0FFEE + 2, shape.vocab, prompt_tokens)
    t0 = time.perf_counter()
    status, logits = model.step_block(prompt, 1)
    prefill_s = time.perf_counter() - t0
    assert status == 0
    token = O.argmax(logits[-1])
    steps = 0
    t0 = time.perf_counter()
    while steps < 4 or (time.perf_counter() - t0 < args.cpu_seconds and steps < 1000):
        status, logits, _ = model.step(np.array([token], dtype=np.int32))
        assert status == 0
        token = O.argmax(logits[0])
        steps += 1
    seconds = time.perf_counter() - t0
    model.close()
    decode_tok_s = steps / seconds
    step_bytes = sum(decode_bytes(L) for L in range(prompt_tokens + 1, prompt_tokens + 1 + steps)) / steps
    log(f"cpu baseline: weights {load:.1f} s, prefill of {prompt_tokens} tokens {prefill_s:.1f} s, "
        f"{steps} decode steps in {seconds:.2f} s ({decode_tok_s:.2f} tok/s)")

    # the two-layer workload end to end: prefill of 16 tokens + 32 greedy tokens
    shape1 = O.gemma_2b_shape(layers=2, max_positions=64)
    small = O.Model(shape1, O.MODE_Q8)
    assert small.fill_synthetic() == 0
    prompt1 = O.prompt_ids(0xC0FFEE + 1, shape1.vocab, 16)
    t0 = time.perf_counter()
    count, ids, _ = small.generate(prompt1, 32, eos=-1)
    config1_s = time.perf_counter() - t0
    small.close()
    log(f"cpu baseline, two-layer workload end to end: {count} tokens in {config1_s:.2f} s")
    host = host_cpu()
    result = {"value": round(decode_tok_s, 3), "unit": "tok/s", "cores": threads, "kind": "port",
              "sample": f"oracle C Q8 decoder ({ORACLE_BUILD}; OpenMP, {threads} threads) at the "
                        f"full Gemma-2B shape ({args.layers} layers): the {prompt_tokens}-token "
                        f"seeded prompt prefilled in blocks ({prefill_s:.1f} s, untimed), then "
                        f"{steps} greedy decode steps timed (positions {prompt_tokens}.."
                        f"{prompt_tokens + steps - 1}, {seconds:.1f} s); host '{host}', "
                        f"nproc {os.cpu_count()}",
              "host": host, "nproc": os.cpu_count(), "build": ORACLE_BUILD,
              "prefill_s": round(prefill_s, 2),
              "config1_end_to_end_s": round(config1_s, 3),
              "config1_tok_s": round(count / config1_s, 2)}
    result["achieved_gbs"] = round(step_bytes * decode_tok_s / 1e9, 2)

    # The reference's own arithmetic (Linear.h:128-357: fp32 activations
    # against Int8Blocks weights dequantized in the product, an fp32 KV
    # cache): the oracle's fp32-activation mode.  It has no blocked prefill,
    # so its sample follows a 16-token prompt; at that length the attention
    # is a sliver of a step whose cost is the 2.66 GB of weights.
    f32 = O.Model(O.gemma_2b_shape(layers=args.layers, max_positions=1024), O.MODE_Q8_PATH_F32)
    assert f32.fill_synthetic() == 0
    prompt16 = O.prompt_ids(0xC0FFEE + 2, shape.vocab, 16)
    status, logits, _ = f32.step(prompt16)
    assert status == 0
    token = O.argmax(logits[-1])
    f32_steps = 0
    t0 = time.perf_counter()
    while f32_steps < 4 or (time.perf_counter() - t0 < args.cpu_seconds and f32_steps < 1000):
        status, logits, _ = f32.step(np.array([token], dtype=np.int32))
        assert status == 0
        token = O.argmax(logits[0])
        f32_steps += 1
    f32_seconds = time.perf_counter() - t0
    f32.close()
    f32_tok_s = f32_steps / f32_seconds
    f32_bytes = sum(decode_bytes(L) for L in range(17, 17 + f32_steps)) / f32_steps
    log(f"cpu baseline, fp32 activations: {f32_steps} decode steps in {f32_seconds:.2f} s "
        f"({f32_tok_s:.2f} tok/s)")
    result["fp32_activations"] = {
        "value": round(f32_tok_s, 3), "unit": "tok/s", "cores": threads,
        "achieved_gbs": round(f32_bytes * f32_tok_s / 1e9, 2),
        "sample": f"oracle C decoder in its fp32-activation mode (the reference's arithmetic: "
                  f"fp32 activations, Int8Blocks weights dequantized in the product, fp32 KV "
                  f"cache; {ORACLE_BUILD}; OpenMP, {threads} threads), {args.layers} layers: a "
                  f"16-token seeded prompt, then {f32_steps} greedy decode steps timed "
                  f"(positions 16..{15 + f32_steps}, {f32_seconds:.1f} s)"}
    return result


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--layers", type=int, default=18)
    ap.add_argument("--threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "0") or 0))
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="timed seconds of the CPU baseline's decode sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the prefill, long-context and lockstep configurations")
    ap.add_argument("--no-graph", action="store_true", help="launch steps without hipGraph replay")
    ap.add_argument("--mode", choices=("all", "decode", "prefill", "long", "batch"), default="all",
                    help="all: the headline decode and the other configurations; the others run "
                         "one configuration alone (for profiles)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device-to-device three times (a kernel of known "
                         "bytes to scale the FETCH_SIZE / WRITE_SIZE counters by)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(batch-1 decode is not sharded across GPUs here)", file=sys.stderr)
        return 2

    import torch
    from huggingfaceeacp_amd import gemma_q8 as G

    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    threads = args.threads if args.threads > 0 else (os.cpu_count() or 1)
    if args.copy_probe > 0:
        src = torch.ones(args.copy_probe << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {args.copy_probe} MiB device-to-device")
        del src, dst
    shape = G.DecoderShape.gemma_2b(layers=args.layers, max_positions=8192, max_step_rows=2048)
    decoder = G.Decoder(shape)
    t0 = time.perf_counter()
    decoder.fill_synthetic(threads)
    log(f"weights generated + quantized on device: {time.perf_counter() - t0:.1f} s")

    if args.mode in ("prefill", "long", "batch"):
        if args.mode == "batch":
            decoder.close()
            out = lockstep_config(args, G, torch, None, shape)
        else:
            run = {"prefill": prefill_config, "long": long_context_config}[args.mode]
            out = run(args, G, torch, decoder, shape)
            decoder.close()
        print(json.dumps({"mode": args.mode, **out}), flush=True)
        return 0

    use_graph = not args.no_graph
    head = headline_decode(args, G, torch, decoder, shape, use_graph)
    configs = None
    if args.mode == "all" and not args.no_configs:
        configs = {"prefill": prefill_config(args, G, torch, decoder, shape),
                   "long_context": long_context_config(args, G, torch, decoder, shape)}
    decoder.close()
    if configs is not None:
        configs["lockstep"] = lockstep_config(args, G, torch, None, shape)
    torch.cuda.synchronize()

    result = {
        "metric": METRIC,
        "value": round(head["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["seconds"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": DATA,
        "config": {"workload": f"Gemma-2B Int8Blocks greedy decode, {args.layers} layers, "
                               f"{args.prompt}-token prompt, {args.steps} timed decode steps, "
                               "fp16 KV cache, batch 1",
                   "layers": args.layers, "prompt_tokens": args.prompt,
                   "decode_steps": args.steps, "graph": use_graph},
        "step_hbm": {"bytes_per_token": int(head["step_bytes"]),
                     "achieved_gbs": round(head["step_gbs"], 1),
                     "frac": round(head["step_gbs"] / HBM_PEAK_GBS, 4)},
        "roofline": head["roofline"],
        "configs": configs,
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(
            args, threads, lambda L: G.algorithmic_decode_bytes(shape, L))
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
