#!/usr/bin/env python3
"""Benchmark of the unmasking generator on one MI355X.

Metric: utterance RTF + unmask steps/s for a 10 s utterance (250 frames at
25 fps, 80 text tokens), 32 steps, CFG 2.0, on the 28-layer Qwen3-0.6B-shaped
backbone with seeded random fp16 weights (synthetic; no checkpoint) and
seeded Gumbel position noise at temperature 5.0.

`--steps K` times K whole utterances: Generator::Generate, i.e. 32
unmasking steps (forward of the packed CFG batch, CFG scoring, top-k
selection) with the inputs already resident on the device and only the
final codes copied back. `value` is unmask steps per second
(32 x utterances / wall time), `ms_per_step` milliseconds per unmasking
step, `ms_per_utterance` per whole utterance, and `utterance_rtf` wall time
per utterance over its seconds of audio.

Other workloads (--workload): 2s, clone (5 s reference voice + 15 s target)
and chunks (four 15 s chunks of long text generated as one batch through
Generator::GenerateBatch; there `value` counts the unmask steps of all four
items and `utterance_rtf` is wall time over the 60 s of audio).

Also reported: the roofline of the dominant kernel (algorithmic FLOPs or
bytes per launch over its HIP-event-timed launch duration on the library
stream, against the bound its arithmetic intensity sets), the algorithmic
HBM bytes of a whole step against its time, and the CPU baseline (the
oracle's float32 restatement of the reference's path, whole unmasking steps
of the same workload on the host's CPUs).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

WORKLOADS = {
    # name: (text tokens, reference frames, target frames)
    "10s": (80, 0, 250),
    "2s": (20, 0, 50),
    "clone": (180, 125, 375),
    # four chunks of long text, batched (4 CFG pairs packed as 8 rows)
    "chunks": (110, 0, 375),
}
ITEMS = {"chunks": 4}  # items generated together (ovg_generate_batch)
DESCRIPTIONS = {
    "10s": "10 s speech",
    "2s": "2 s speech",
    "clone": "15 s speech cloning a 5 s reference",
    "chunks": "4 x 15 s chunks of long text batched",
}


def make_input(ov, text, reference, target, seed=42):
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, 151936, size=text)
    refc = rng.integers(0, 1024, size=(8, reference)) if reference else None
    return ov.ConditionalInput.build(tokens, refc, reference, target)


def host_cpu():
    """(model name, logical CPUs this process may run on, threads to use):
    every CPU in the affinity mask, capped by OMP_NUM_THREADS where it is set
    (on a host shared by several GPUs, typically one GPU's share of it)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    available = len(os.sched_getaffinity(0))
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return model, available, min(available, cap) if cap > 0 else available


def cpu_baseline(cfg, x, decoding, min_seconds):
    """The oracle (float32) timed on whole unmasking steps of the workload
    (forward, score and select), as many as fit `min_seconds` (at least
    two), on every CPU of this process's share of the host."""
    import oracle
    model_name, available, threads = host_cpu()
    oracle.lib().orc_set_threads(threads)
    t0 = time.perf_counter()
    model = oracle.Model(cfg, 1234)
    setup = time.perf_counter() - t0
    ids = np.ascontiguousarray(x.ids)
    C, F, V = 8, x.target_frames, 1025
    sel = oracle.Selector(decoding.layer_penalty, decoding.position_temperature, 42)
    codes = np.full(C * F, 1024, dtype=np.int32)
    schedule = [c for c in oracle.unmask_schedule(C * F, 32, decoding.t_shift) if c]
    t0 = time.perf_counter()
    steps = 0
    while steps < len(schedule) and (steps < 2 or time.perf_counter() - t0 < min_seconds):
        logits = model.forward(ids, x.audio_start, F)
        pred, conf = oracle.score(logits, F, C, V, 1024, decoding.guidance)
        sel.fill(schedule[steps], C, F, pred, conf, 1024, codes)
        ids[:, -F:] = codes.reshape(C, F)
        steps += 1
    elapsed = time.perf_counter() - t0
    return {"value": steps / elapsed, "unit": "unmask steps/s", "cores": threads,
            "kind": "port", "cpu_model": model_name, "cpus_available": available,
            "sample": f"the first {steps} of the {len(schedule)} unmasking steps of one "
                      f"{F}-frame utterance (forward of {x.length + F} packed rows, score, "
                      f"select, write-back), float32 oracle on {threads} threads of "
                      f"{model_name}, {elapsed:.1f} s; weight synthesis {setup:.1f} s "
                      f"excluded",
            "utterance_rtf_extrapolated": (elapsed / steps * len(schedule)) / (F / 25.0)}


def bench_codec(args, torch):
    """The audio decoder on the workload's frames: codes resident on the
    device, audio left there (Codec::Decode without the host copies)."""
    import omnivoice_amd as ov
    cfg = ov.codec_released_config()
    frames = WORKLOADS[args.workload][2] * ITEMS.get(args.workload, 1)
    codec = ov.Codec.synthetic(cfg, 1234)
    rng = np.random.default_rng(42)
    codes_host = rng.integers(0, 1024, size=(8, frames)).astype(np.int32)
    codes = torch.from_numpy(codes_host).cuda()
    audio = torch.empty(codec.samples(frames), dtype=torch.float32, device="cuda")
    for _ in range(args.warmup):
        codec.decode_device(codes, audio)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        codec.decode_device(codes, audio)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    seconds = frames / 25.0
    stats = codec.profile(frames, repeats=args.profile_repeats)
    kernels = {n: {"launches": s["launches"], "avg_us": s["total_ms"] / s["launches"] * 1e3,
                   "tflops": s["flops"] / (s["total_ms"] * 1e-3) / 1e12 if s["flops"] else None}
               for n, s in stats.items()}
    dominant = max(stats, key=lambda n: stats[n]["total_ms"])
    d = stats[dominant]
    achieved = d["flops"] / (d["total_ms"] * 1e-3) / 1e12
    total_flops = sum(s["flops"] for s in stats.values()) / args.profile_repeats
    result = {
        "metric": f"audio decode, {seconds:g} s of 24 kHz audio ({frames} frames), 1 GPU",
        "value": seconds * args.steps / elapsed,
        "unit": "audio seconds decoded per second",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded decoder weights, uniform codes)",
        "config": {"workload": f"{args.workload}: decode of {frames} frames x 8 codebooks "
                               f"to {codec.samples(frames)} samples",
                   "decoder": "Higgs Audio v2 DAC decoder (1024 ch, upsampling 8 5 4 2 3)",
                   "parallelism": "single GPU"},
        "decode_rtf": (elapsed / args.steps) / seconds,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_FP32_TFLOPS, "traffic": None,
                     "kernel": dominant,
                     "avg_launch_us": d["total_ms"] / d["launches"] * 1e3},
        "decode_tflops": total_flops / (elapsed / args.steps) / 1e12,
        "kernels": kernels,
    }
    if args.cpu_seconds > 0:
        import oracle
        model_name, _, threads = host_cpu()
        oracle.lib().orc_set_threads(threads)
        model = oracle.Codec(oracle.codec_released_config(), 1234)
        sample = codes_host[:, :25]
        t0 = time.perf_counter()
        model.decode(sample)
        cpu = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": 1.0 / cpu, "unit": "audio seconds decoded per second",
                                  "cores": threads, "kind": "port", "cpu_model": model_name,
                                  "sample": "1 s (25 frames) decoded by the float32 oracle "
                                            "(double sums); table synthesis excluded"}
    print(json.dumps(result), flush=True)


def bench_encode(args, torch):
    """The audio encoder on the workload's length of reference audio: samples
    resident on the device, codes left there (Codec::Encode without the host
    copies)."""
    import omnivoice_amd as ov
    cfg = ov.encoder_released_config()
    frames = WORKLOADS[args.workload][2] * ITEMS.get(args.workload, 1)
    length = frames * cfg["frame_samples"]
    encoder = ov.Encoder.synthetic(cfg, 1234)
    t = np.arange(length)
    rng = np.random.default_rng(42)
    host = (0.3 * np.sin(2 * np.pi * 220 * t / 24000) * (0.5 + 0.5 * np.sin(t / 900))
            + 0.03 * rng.standard_normal(length)).astype(np.float32)
    samples = torch.from_numpy(host).cuda()
    codes = torch.empty((cfg["codebooks"], frames), dtype=torch.int32, device="cuda")
    for _ in range(args.warmup):
        encoder.encode_device(samples, codes)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        encoder.encode_device(samples, codes)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    seconds = length / 24000.0
    stats = encoder.profile(length, repeats=args.profile_repeats)
    kernels = {n: {"launches": s["launches"], "avg_us": s["total_ms"] / s["launches"] * 1e3,
                   "total_ms": s["total_ms"] / args.profile_repeats,
                   "tflops": s["flops"] / (s["total_ms"] * 1e-3) / 1e12 if s["flops"] else None}
               for n, s in stats.items()}
    dominant = max(stats, key=lambda n: stats[n]["total_ms"])
    d = stats[dominant]
    achieved = d["flops"] / (d["total_ms"] * 1e-3) / 1e12
    total_flops = sum(s["flops"] for s in stats.values()) / args.profile_repeats
    result = {
        "metric": f"audio encode, {seconds:g} s of 24 kHz reference audio ({frames} frames), "
                  f"1 GPU",
        "value": seconds * args.steps / elapsed,
        "unit": "audio seconds encoded per second",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded encoder weights, a modulated tone with noise)",
        "config": {"workload": f"{args.workload}: encode of {length} samples to {frames} "
                               f"frames x 8 codebooks",
                   "encoder": "Higgs Audio v2 tokenizer encoder (HuBERT base at 16 kHz, "
                              "DAC encoder 64 ch, strides 8 5 4 2 3, RVQ 8 x 1024)",
                   "parallelism": "single GPU"},
        "encode_rtf": (elapsed / args.steps) / seconds,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_FP32_TFLOPS, "traffic": None,
                     "kernel": dominant,
                     "avg_launch_us": d["total_ms"] / d["launches"] * 1e3},
        "encode_tflops": total_flops / (elapsed / args.steps) / 1e12,
        "kernels": kernels,
    }
    if args.cpu_seconds > 0:
        import oracle
        model_name, _, threads = host_cpu()
        oracle.lib().orc_set_threads(threads)
        model = oracle.Encoder(oracle.encoder_released_config(), 1234)
        sample = host[:24000]
        t0 = time.perf_counter()
        model.encode(sample)
        cpu = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": 1.0 / cpu, "unit": "audio seconds encoded per second",
                                  "cores": threads, "kind": "port", "cpu_model": model_name,
                                  "sample": "1 s (25 frames) encoded by the float32 oracle "
                                            "(double sums); weight synthesis excluded"}
    print(json.dumps(result), flush=True)


def gemm_compare(args, torch):
    """The vendor library at the backbone's GEMM shapes, as a speed
    comparator: torch.matmul (hipBLASLt) fp16 x fp16 -> fp16, 28 distinct
    weight matrices per shape (one per layer, so weights stream from HBM as
    in a step) replayed in a HIP graph; per-GEMM time = graph time / 28."""
    shapes = [("qkv", 4096, 1024), ("gate_up", 6144, 1024), ("o", 1024, 2048),
              ("down", 1024, 3072)]
    rows = {"C2": 120, "C3": 580, "C4": 1055, "C5": 3440}
    out = []
    for config, m in rows.items():
        for name, n, k in shapes:
            x = torch.randn(m, k, device="cuda", dtype=torch.float16)
            ws = [torch.randn(n, k, device="cuda", dtype=torch.float16) * 0.02
                  for _ in range(28)]
            ys = [torch.empty(m, n, device="cuda", dtype=torch.float16) for _ in range(28)]
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for l in range(28):
                    torch.matmul(x, ws[l].t(), out=ys[l])
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for l in range(28):
                    torch.matmul(x, ws[l].t(), out=ys[l])
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            reps = 20
            a.record()
            for _ in range(reps):
                g.replay()
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / (reps * 28)
            out.append({"config": config, "gemm": name, "m": m, "n": n, "k": k,
                        "us": us, "tflops": 2.0 * m * n * k / us / 1e6})
            del ws, ys, g
    print(json.dumps({"comparator": "torch.matmul (hipBLASLt), fp16 out, HIP graph of 28",
                      "torch": torch.__version__, "rows": out}), flush=True)


def linear_tiles(specs, torch):
    """Five launches of the packed-weight GEMM per shape with the tile
    forced (fp32 stores, seeded fp16 operands), nothing timed: a fixed
    workload for rocprofv3 counter passes over one kernel kind each."""
    import omnivoice_amd as ov
    rng = np.random.default_rng(0)
    for spec in specs:
        shape, tile = spec.split(":")
        m, n, k = (int(v) for v in shape.split("x"))
        r, c = (int(v) for v in tile.split("x"))
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).cuda()
        w = torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float16)).cuda()
        y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        for _ in range(5):
            ov.op_linear_packed(x, w, y, tile_rows=r, tile_cols=c)
        torch.cuda.synchronize()
        print(json.dumps({"linear": spec, "launches": 5}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200,
                    help="utterances timed (each one Generate call of 32 unmasking steps; "
                         "200 at 10 s keep the GPU busy for ~12 s)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="10s", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="seconds of whole unmasking steps timed for the CPU baseline "
                         "(0 skips it)")
    ap.add_argument("--profile-repeats", type=int, default=3)
    ap.add_argument("--codec", action="store_true",
                    help="benchmark the audio decoder on the workload's frames instead")
    ap.add_argument("--encode", action="store_true",
                    help="benchmark the audio encoder on the workload's length of audio")
    ap.add_argument("--gemm-compare", action="store_true",
                    help="time the vendor GEMM (torch.matmul) at the backbone's shapes")
    ap.add_argument("--linear-tiles", nargs="*", default=None, metavar="MxNxK:RxC",
                    help="only run ovg_op_linear_packed five times per shape with the "
                         "tile forced (e.g. 3440x4096x1024:256x256), for counter "
                         "passes, and exit")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only copy this many MiB device to device 3 times (a "
                         "copy kernel of known size for calibrating memory "
                         "counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this library runs on one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is design-only)"}))
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        raise SystemExit("no GPU visible")
    if args.copy_calibration_mb > 0:
        n = args.copy_calibration_mb << 20
        src = torch.full((n,), 1, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "copies": 3}), flush=True)
        return
    if args.linear_tiles is not None:
        linear_tiles(args.linear_tiles, torch)
        return
    if args.codec:
        bench_codec(args, torch)
        return
    if args.encode:
        bench_encode(args, torch)
        return
    if args.gemm_compare:
        gemm_compare(args, torch)
        return
    import omnivoice_amd as ov

    cfg = ov.released_config()
    text, reference, target = WORKLOADS[args.workload]
    items = ITEMS.get(args.workload, 1)
    xs = [make_input(ov, text, reference, target, seed=42 + j) for j in range(items)]
    x = xs[0]
    decoding = ov.DecodingConfig(steps=32, guidance=2.0, t_shift=0.1,
                                 layer_penalty=5.0, position_temperature=5.0)
    t0 = time.perf_counter()
    gen = ov.Generator.synthetic(cfg, 1234)
    load_s = time.perf_counter() - t0
    executed = sum(1 for c in ov.unmask_schedule(8 * target, 32, 0.1) if c)

    def run(i):
        if items == 1:
            gen.generate(x, decoding, seed=42 + i)
        else:
            gen.generate_batch(xs, decoding, seeds=[42 + i * items + j for j in range(items)])

    for i in range(args.warmup):
        run(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    # generate returns the codes on the host, so every utterance ends
    # synchronised: its own wall time needs no extra synchronisation.
    marks = [t0]
    for i in range(args.steps):
        run(i)
        marks.append(time.perf_counter())
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_utterance = elapsed / args.steps * 1e3
    each_ms = sorted((b - a) * 1e3 for a, b in zip(marks, marks[1:]))
    steps_per_s = executed * items * args.steps / elapsed
    rtf = (elapsed / args.steps) / (items * target / 25.0)

    stats = gen.profile(xs if items > 1 else x, repeats=args.profile_repeats)
    kernels = {}
    for name, s in stats.items():
        avg = s["total_ms"] / s["launches"]
        kernels[name] = {"launches": s["launches"], "avg_us": avg * 1e3,
                         "share": 0.0,
                         "tflops": s["flops"] / (s["total_ms"] * 1e-3) / 1e12
                         if s["flops"] else None,
                         "gbs": s["bytes"] / (s["total_ms"] * 1e-3) / 1e9}
    total_ms = sum(s["total_ms"] for s in stats.values())
    for name, s in stats.items():
        kernels[name]["share"] = s["total_ms"] / total_ms
    dominant = max(stats, key=lambda n: stats[n]["total_ms"])
    d = stats[dominant]
    per_launch_ms = d["total_ms"] / d["launches"]
    # The bound is the one the kernel's arithmetic intensity puts it under:
    # below the ridge point (peak FLOP/s over peak bytes/s, 312.5 FLOP/B)
    # HBM, above it the matrix cores (the 2 s workload's GEMMs stream their
    # weights; the 10 s, clone and chunk GEMMs are compute-bound).
    intensity = d["flops"] / d["bytes"] if d["bytes"] else float("inf")
    ridge = PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    if d["flops"] and intensity >= ridge:
        achieved = d["flops"] / d["launches"] / (per_launch_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP16_TFLOPS,
                    "unit": "TFLOP/s", "frac": achieved / PEAK_FP16_TFLOPS}
    else:
        achieved = d["bytes"] / d["launches"] / (per_launch_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS}
    roofline.update({"traffic": None, "kernel": dominant,
                     "avg_launch_us": per_launch_ms * 1e3,
                     "algorithmic_flops": d["flops"] / d["launches"],
                     "algorithmic_bytes": d["bytes"] / d["launches"],
                     "intensity_flop_per_byte": intensity})
    # HBM bytes per launch of the dominant kernel, from the calibrated
    # FETCH_SIZE / WRITE_SIZE counter runs summarised under profiles/.
    traffic_path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if os.path.exists(traffic_path):
        with open(traffic_path) as f:
            measured = json.load(f).get(args.workload, {}).get(dominant)
        if measured:
            roofline["traffic"] = measured["bytes"]
            roofline["traffic_source"] = "profiles/" + measured["source"]
    gemm_ms = sum(s["total_ms"] for n, s in stats.items() if n.startswith("gemm_")
                  and n != "gemm_audio_heads")
    gemm_flops = sum(s["flops"] for n, s in stats.items() if n.startswith("gemm_")
                     and n != "gemm_audio_heads")

    # Algorithmic HBM bytes of one unmasking step: every fp16 weight read
    # once, the logits written once (2 F rows of 8 x 1025 floats per item)
    # and the embedding rows (R real packed rows of 1024 floats).
    h, inter = cfg["hidden_size"], cfg["intermediate_size"]
    qkv_n = (cfg["heads"] + 2 * cfg["kv_heads"]) * 128
    width = cfg["audio_codebooks"] * cfg["audio_vocab_size"]
    backbone_params = cfg["layers"] * (qkv_n * h + h * cfg["heads"] * 128 + 3 * inter * h)
    real_rows = items * (text + reference + 2 * target)
    step_bytes = (2 * (backbone_params + width * h) + items * 2 * target * width * 4
                  + real_rows * h * 4)
    kernel_bytes = sum(s["bytes"] for s in stats.values()) / args.profile_repeats
    ms_per_unmask_step = elapsed / (args.steps * executed) * 1e3
    result = {
        "metric": f"utterance RTF + unmask steps/s, {DESCRIPTIONS[args.workload]}, "
                  f"32 steps, CFG 2.0, 1 GPU",
        "value": steps_per_s,
        "unit": "unmask steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_unmask_step,
        "step_unit": f"ms_per_step is per unmasking step (one forward of the packed batch, "
                     f"CFG score and top-k select); --steps counts utterances of "
                     f"{executed} unmasking steps each",
        "ms_per_utterance": ms_per_utterance,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0, 0.02) fp16 weights, uniform text ids, masked target)",
        "config": {"workload": f"{args.workload}: {items} x ({text} text tokens, {reference} "
                               f"reference frames, {target} masked target frames), "
                               f"{items} CFG pair(s) packed as "
                               f"{items * (text + reference + 2 * target)} rows, "
                               f"32 steps, guidance 2.0, position temperature 5.0"
                               if items > 1 else
                               f"{args.workload}: {text} text tokens, {reference} "
                               f"reference frames, {target} masked target frames, "
                               f"CFG pair packed as {text + reference + 2 * target} rows, "
                               f"32 steps, guidance 2.0, position temperature 5.0",
                   "backbone": "28 x Qwen3 (hidden 1024, 16q/8kv x 128, FFN 3072)",
                   "parallelism": "single GPU"},
        "utterance_rtf": rtf,
        "utterance_ms": {"median": each_ms[len(each_ms) // 2], "min": each_ms[0],
                         "max": each_ms[-1]},
        "unmask_steps_per_utterance": executed,
        "roofline": roofline,
        "backbone_gemm_tflops": gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms else None,
        "eager_step_ms": total_ms / args.profile_repeats,
        "step_hbm": {"algorithmic_bytes": step_bytes,
                     "achieved_gbs": step_bytes / (ms_per_unmask_step * 1e-3) / 1e9,
                     "frac": step_bytes / (ms_per_unmask_step * 1e-3) / 1e9 / PEAK_HBM_GBS,
                     "kernels_algorithmic_bytes": kernel_bytes},
        "kernels": kernels,
        "load_s": load_s,
    }
    if args.cpu_seconds > 0 and items == 1:
        result["cpu_baseline"] = cpu_baseline(cfg, x, decoding, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
