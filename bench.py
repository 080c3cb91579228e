#!/usr/bin/env python3
"""Gemma-2B Int8Blocks decode throughput on one MI355X.

Workload (the headline decode configuration): the full Gemma-2B shape (18
layers, width 2048, 8 query heads / 1 KV head of 256, FFN 16384, vocabulary
256000 with the tied embedding), seeded N(0, 0.02) weights (norms N(0, 0.1))
quantized to Int8Blocks, a 512-token seeded uniform prompt, greedy decode with
an fp16 KV cache.  A step is one decode token: embed, 18 layers, final norm,
the tied lm_head over 256000 rows and the on-device argmax that feeds the next
step.  The prefill is untimed; W warmup decode steps run in a separate
sequence; then exactly K decode steps are timed after a fresh 512-token
prefill, bracketed by device synchronisation.

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
# HBM bytes a launch moves, from two rocprofv3 counter passes over the decode
# kernels: FETCH_SIZE scaled by what it reads for a 256 MiB copy (x 1.99977),
# plus WRITE_SIZE (the passes and their commands are in
# profiles/decode_kernels_gemma2b_hbm_traffic.md).  A kernel change
# re-measures these.
MEASURED_TRAFFIC = {"gate_up": 71572184, "lm_head": 558419832, "down": 35954732}
METRIC = "Gemma-2B Q8_0 decode tok/s (b=1, ctx 512) + % of HBM roofline"
STAGE_LABELS = {
    "gate_up": "gateup_geglu_kernel (post-attention norm + gate|up 2048 -> 2x16384 + GeGLU + Q8)",
    "lm_head": "lmhead_argmax_kernel (tied lm_head 2048 -> 256000 + first-maximum fold)",
    "down": "q8_matvec_kernel<1,4,2> (down 16384 -> 2048 + residual)",
}


def log(*args):
    print(*args, file=sys.stderr, flush=True)


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


def cpu_baseline(layers: int, seconds_target: float, threads: int) -> dict:
    """The oracle's Q8 decoder (C, OpenMP over the host cores): a bounded
    sample of the same decode loop, after a short untimed prefill."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    O.lib()
    prompt_tokens, max_positions = 32, 1024
    shape = O.gemma_2b_shape(layers=layers, max_positions=max_positions)
    model = O.Model(shape, O.MODE_Q8)
    t0 = time.perf_counter()
    assert model.fill_synthetic() == 0
    load = time.perf_counter() - t0
    prompt = O.prompt_ids(0xC0FFEE + 2, shape.vocab, prompt_tokens)
    status, logits, _ = model.step(prompt)
    assert status == 0
    token = O.argmax(logits[-1])
    steps = 0
    t0 = time.perf_counter()
    while steps < 8 or (time.perf_counter() - t0 < seconds_target
                        and prompt_tokens + steps < max_positions - 1):
        status, logits, _ = model.step(np.array([token], dtype=np.int32))
        assert status == 0
        token = O.argmax(logits[0])
        steps += 1
    seconds = time.perf_counter() - t0
    model.close()
    log(f"cpu baseline: weights {load:.1f} s, {steps} steps in {seconds:.2f} s")
    return {"value": round(steps / seconds, 3), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle C Q8 decoder (OpenMP, {threads} threads) at the full Gemma-2B "
                      f"shape ({layers} layers), {prompt_tokens}-token seeded prompt prefilled "
                      f"untimed, then {steps} greedy decode steps timed (positions "
                      f"{prompt_tokens}..{prompt_tokens + steps - 1}, about {seconds:.0f} s); host "
                      f"'{platform.processor() or platform.machine()}'"}


PREFILL_METRIC = "Gemma-2B Q8_0 prefill tok/s (b=1, 2048-token prompt) + int8 MFMA utilisation"
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA


def prefill_bench(args, G, torch) -> dict:
    """The prefill workload: a 2048-token seeded prompt through all 18 layers
    as one step (every linear an int8 MFMA GEMM of M = 2048), logits of the
    last row only; W untimed prefills, then K timed."""
    rows = args.prompt
    shape = G.DecoderShape.gemma_2b(layers=args.layers, max_positions=max(rows + 1, 2048),
                                    max_step_rows=rows)
    decoder = G.Decoder(shape)
    threads = args.threads if args.threads > 0 else (os.cpu_count() or 1)
    decoder.fill_synthetic(threads)
    prompt = G.prompt_ids(0xC0FFEE + 3, shape.vocab, rows).astype(np.uint32)
    ids = torch.from_numpy(prompt.copy()).to("cuda")
    logits = torch.empty(shape.vocab, dtype=torch.float32, device="cuda")

    def once():
        decoder.begin_sequence()
        decoder.step(ids.data_ptr(), rows, logits.data_ptr(), 1)

    for _ in range(args.warmup):
        once()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        once()
    torch.cuda.synchronize()
    seconds = (time.perf_counter() - t0) / args.steps
    linear = args.layers * (shape.width * (shape.query_width + 2 * shape.kv_width)
                            + shape.query_width * shape.width
                            + 2 * shape.width * shape.intermediate
                            + shape.intermediate * shape.width)
    int_ops = 2 * rows * linear + 2 * shape.width * shape.vocab  # lm_head: the last row
    tops = int_ops / seconds / 1e12
    log(f"prefill of {rows} tokens: {seconds * 1e3:.2f} ms, {int_ops / 1e12:.3f} T int8 ops, "
        f"{tops:.1f} TOP/s")
    return {
        "metric": PREFILL_METRIC, "value": round(rows / seconds, 1), "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(seconds * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded N(0,0.02) weights / N(0,0.1) norms quantized to Int8Blocks, "
                "seeded uniform prompt ids",
        "config": {"workload": f"Gemma-2B Int8Blocks prefill, {args.layers} layers, "
                               f"{rows}-token prompt as one step, last-row logits",
                   "layers": args.layers, "prompt_tokens": rows},
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": None,
                     "counted": "2 M K N int8 ops over every linear plus the last row's lm_head; "
                                "attention's fp64 work not counted"},
        "cpu_baseline": None,
    }


BATCH_METRIC = "Gemma-2B Q8_0 lockstep decode tok/s (16 sequences x (1024 prompt + 128 decode))"


def batch_stage_bytes(shape, stage: str, rows: int) -> int:
    """Algorithmic HBM bytes of one lockstep product launch: the Int8Blocks
    weights once, the rows' Q8 inputs and fp32 outputs (read and written for
    a residual)."""
    w, f, v = shape.width, shape.intermediate, shape.vocab
    q8 = lambda n: n * 17 // 16  # noqa: E731
    if stage == "gate_up":  # GeGLU fused: Q8 rows in, GeGLU's Q8 rows out
        return q8(2 * f * w) + rows * (q8(w) + q8(f))
    if stage == "lm_head":
        return q8(v * w) + rows * (q8(w) + v * 4)
    if stage == "down":
        return q8(f * w) + rows * (q8(f) + 2 * w * 4)
    raise ValueError(stage)


def batch_bench(args, G, torch) -> dict:
    """The lockstep workload: S sequences of seeded 1024-token prompts
    (prefilled one by one, untimed), W untimed lockstep steps, then the
    sequences are prefilled again and exactly K lockstep steps are timed."""
    S, prompt_len = args.sequences, args.prompt
    steps = args.steps
    shape = G.DecoderShape.gemma_2b(layers=args.layers, max_positions=prompt_len + steps + args.warmup + 1,
                                    max_step_rows=256)
    decoder = G.Decoder(shape)
    threads = args.threads if args.threads > 0 else (os.cpu_count() or 1)
    decoder.fill_synthetic(threads)
    batch = G.Batch(decoder, S)
    prompts = [G.prompt_ids(0xC0FFEE + 5 + 1000 * s, shape.vocab, prompt_len) for s in range(S)]

    def prefill_all():
        t = time.perf_counter()
        for s, prompt in enumerate(prompts):
            batch.prefill(s, prompt)
        return time.perf_counter() - t

    prefill_all()
    batch.decode(args.warmup, use_graph=True)
    prefill_s = prefill_all()
    log(f"prefill of {S} x {prompt_len} tokens: {prefill_s * 1e3:.1f} ms")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    batch.decode(steps, use_graph=True)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    tok_s = S * steps / seconds
    step_bytes = sum(G.algorithmic_batch_step_bytes(shape, [prompt_len + k + 1] * S)
                     for k in range(steps)) / steps
    step_gbs = step_bytes * steps / seconds / 1e9
    log(f"lockstep: {tok_s:.1f} tok/s, {seconds / steps * 1e3:.3f} ms/step, {step_gbs:.0f} GB/s of "
        f"{step_bytes / 1e9:.4f} GB/step; sequence 0 ids {list(batch.tokens(0, prompt_len, 6))}")

    # stage breakdown and the dominant product's launch duration: eager steps
    # with every launch group bracketed by HIP events
    prefill_all()
    timed = min(steps, 32)
    decoder.set_timing(True)
    batch.decode(timed, use_graph=False)
    timing = decoder.timing()
    decoder.set_timing(False)
    total_ms = sum(ms for ms, _ in timing.values())
    for name, (ms, n) in sorted(timing.items(), key=lambda kv: -kv[1][0]):
        if n:
            log(f"  {name:10s} {ms / timed * 1e3:8.1f} us/step  {n // timed:3d} launches/step"
                f"  {100 * ms / total_ms:5.1f} %")
    dominant = max(("gate_up", "lm_head", "down"), key=lambda k: timing[k][0])
    ms, launches = timing[dominant]
    per_launch_s = ms / launches / 1e3
    launch_bytes = batch_stage_bytes(shape, dominant, S)
    achieved = launch_bytes / per_launch_s / 1e9
    labels = {"gate_up": "q8_rows_kernel (gate|up 2048 -> 2x16384 + GeGLU + Q8, 16 rows)",
              "lm_head": "q8_rows_kernel (tied lm_head 2048 -> 256000, 16 rows)",
              "down": "q8_rows_kernel (down 16384 -> 2048 + residual, 16 rows)"}
    batch.close()
    return {
        "metric": BATCH_METRIC, "value": round(tok_s, 1), "unit": "tok/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(seconds / steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded N(0,0.02) weights / N(0,0.1) norms quantized to Int8Blocks, "
                "seeded uniform prompt ids",
        "config": {"workload": f"Gemma-2B Int8Blocks lockstep greedy decode, {args.layers} layers, "
                               f"{S} sequences x ({prompt_len} prompt + {steps} timed steps), "
                               "fp16 KV caches",
                   "layers": args.layers, "sequences": S, "prompt_tokens": prompt_len,
                   "decode_steps": steps, "graph": True},
        "step_hbm": {"bytes_per_step": int(step_bytes), "achieved_gbs": round(step_gbs, 1),
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": labels[dominant], "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_launch": launch_bytes,
                     "avg_launch_us": round(per_launch_s * 1e6, 2)},
        "cpu_baseline": None,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--layers", type=int, default=18)
    ap.add_argument("--threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "0") or 0))
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="timed seconds of the CPU baseline's decode sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-graph", action="store_true", help="launch steps without hipGraph replay")
    ap.add_argument("--flow", action="store_true",
                    help="decode steps as one dataflow launch a token")
    ap.add_argument("--persistent", action="store_true",
                    help="decode steps as one persistent launch a token (one workgroup a compute unit)")
    ap.add_argument("--mode", choices=("decode", "prefill", "batch"), default="decode",
                    help="decode: the headline decode loop; prefill: the 2048-token prefill "
                         "(use with --prompt 2048); batch: lockstep decode of --sequences "
                         "sequences (use with --prompt 1024 --steps 128)")
    ap.add_argument("--sequences", type=int, default=16, help="sequences of --mode batch")
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
    if args.mode == "prefill":
        print(json.dumps(prefill_bench(args, G, torch)), flush=True)
        return 0
    if args.mode == "batch":
        print(json.dumps(batch_bench(args, G, torch)), flush=True)
        return 0
    threads = args.threads if args.threads > 0 else (os.cpu_count() or 1)
    if args.copy_probe > 0:
        src = torch.ones(args.copy_probe << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {args.copy_probe} MiB device-to-device")
        del src, dst
    max_positions = 8192
    shape = G.DecoderShape.gemma_2b(layers=args.layers, max_positions=max_positions,
                                    max_step_rows=512)
    decoder = G.Decoder(shape)
    t0 = time.perf_counter()
    decoder.fill_synthetic(threads)
    log(f"weights generated + quantized on device: {time.perf_counter() - t0:.1f} s")
    prompt = G.prompt_ids(0xC0FFEE + 2, shape.vocab, args.prompt)
    use_graph = not args.no_graph
    decoder.set_flow(args.flow)
    decoder.set_persistent(args.persistent)

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
    lengths = range(first_l, first_l + args.steps)
    step_bytes = sum(G.algorithmic_decode_bytes(shape, L) for L in lengths) / args.steps
    step_gbs = step_bytes * tok_s / 1e9
    tokens = decoder.tokens(args.prompt, args.steps + 1)
    log(f"decode: {tok_s:.1f} tok/s, {seconds / args.steps * 1e3:.3f} ms/step, "
        f"{step_gbs:.0f} GB/s of {step_bytes / 1e9:.4f} GB/token; first ids {list(tokens[:6])}")

    # the stage breakdown: every launch group of K more steps bracketed by HIP
    # events on the decoder's stream (the event packets add about a
    # microsecond to each bracket)
    decoder.set_flow(False)
    decoder.set_persistent(False)
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
                "traffic": MEASURED_TRAFFIC.get(dominant), "bytes_per_launch": launch_bytes,
                "avg_launch_us": round(per_launch_s * 1e6, 2)}

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(seconds / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded N(0,0.02) weights / N(0,0.1) norms quantized to Int8Blocks, "
                "seeded uniform prompt ids",
        "config": {"workload": f"Gemma-2B Int8Blocks greedy decode, {args.layers} layers, "
                               f"{args.prompt}-token prompt, {args.steps} timed decode steps, "
                               "fp16 KV cache, batch 1",
                   "layers": args.layers, "prompt_tokens": args.prompt,
                   "decode_steps": args.steps, "graph": use_graph, "flow": args.flow,
                   "persistent": args.persistent},
        "step_hbm": {"bytes_per_token": int(step_bytes), "achieved_gbs": round(step_gbs, 1),
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.layers, args.cpu_seconds, threads)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
