"""Decode benchmark of the MI355X Qwen3-ASR text decoder (BASELINE metric, one GPU).

    python bench.py [--gpus 1] [--steps 64] [--warmup 8] [--config 3] [--no-cpu-baseline]

Workload (config 3): Qwen3-ASR-1.7B decoder, seeded N(0, 0.02) f32 weights, f16 KV cache, prefill of
3913 positions (3900 audio rows N(0, 1) + 13 random prompt ids), then greedy decode at ~4k context.
A step is one decode token: embedding gather, 28 layers (fused K/V append, split-K attention, f32
GEMVs), LM head and device argmax.  value = decode tokens/s over exactly --steps steps, inputs and
weights resident in HBM, bracketed by device synchronisation.

Also reported: the decode attention's achieved HBM bandwidth (algorithmic bytes 4096 * L + 16384 per
layer call, timed with HIP events on the decoder stream), prefill time, and the CPU oracle's decode
rate on a bounded sample (cpu_baseline, kind "port").
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "qwenasr.cpp_amd")]

METRIC = "decode tok/s + KV-attn HBM GB/s (% of peak), Qwen3-ASR-1.7B decoder, 1 GPU"
HBM_PEAK_GBS = 8000.0


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(model, length: int, steps: int):
    """Oracle decode steps of the same model at the same context (cache rows N(0, 1), f16)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import qa_oracle as orc
    import qwenasr_amd as qa

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = min(cores, 16)
    orc.set_threads(cores)
    om = orc.OracleModel.from_product_model(model)
    c = model.cfg
    cache = om.cache(length + steps + 1, f16=True)
    n = c.n_layers * c.n_kv_heads * length * c.head_dim
    k = qa.synth_normal(n, qa.SEED_KV, "bench.cpu.k").reshape(c.n_layers, c.n_kv_heads, length, c.head_dim)
    v = qa.synth_normal(n, qa.SEED_KV, "bench.cpu.v").reshape(c.n_layers, c.n_kv_heads, length, c.head_dim)
    cache.fill(k, v, length)
    del k, v
    om.decode_steps(cache, 1234, 1)                    # warm caches and thread pool
    t0 = time.perf_counter()
    om.decode_steps(cache, 1234, steps)
    dt = time.perf_counter() - t0
    return dict(value=round(steps / dt, 4), unit="tok/s", cores=cores, kind="port",
                sample=f"{steps} oracle decode steps of the 1.7B decoder at context {length + 1}..{length + steps + 1}, "
                       f"f16 cache, {dt:.1f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", type=int, default=3, choices=[2, 3])
    ap.add_argument("--profile-steps", type=int, default=16)
    ap.add_argument("--cpu-steps", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the KV-cache path shards by "
              "KV head or by stream, see DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import qwenasr_amd as qa
    from qwenasr_amd import configs

    assert qa.device_count() > 0, "bench.py needs a HIP device"
    w = configs.CONFIGS[args.config]
    t0 = time.perf_counter()
    model = qa.Model(w.size, n_layers=w.n_layers)
    x = qa.prompt_input(model, w.audio_tokens, w.prompt_tokens)
    log(f"synthetic {w.size.name} built in {time.perf_counter() - t0:.1f}s")
    max_seq = w.prompt + args.warmup + args.steps + args.profile_steps + 2
    dec = qa.Decoder(model, 1, max_seq, w.cache_type)
    log(f"decoder ready (weights + {max_seq}-position f16 cache on device)")

    qa.check(qa.lib.qa_device_synchronize())
    t0 = time.perf_counter()
    logits = dec.forward(x, 0)
    prefill_ms = (time.perf_counter() - t0) * 1e3
    first = int(np.argmax(logits))
    log(f"prefill {w.prompt} positions: {prefill_ms:.1f} ms")

    ids = dec.decode_streams(np.array([first], np.int32), args.warmup) if args.warmup else np.array([[first]])
    last = int(ids[-1, 0])
    qa.check(qa.lib.qa_device_synchronize())
    ctx0 = dec.cur_len(0)
    t0 = time.perf_counter()
    ids = dec.decode_streams(np.array([last], np.int32), args.steps)
    qa.check(qa.lib.qa_device_synchronize())
    dt = time.perf_counter() - t0
    log(f"timed {args.steps} decode steps at context {ctx0}..{ctx0 + args.steps}: {dt * 1e3:.1f} ms")

    # attention roofline: HIP events around every decode-attention call on the decoder stream
    dec.profile(True)
    dec.profile_reset()
    ctx1 = dec.cur_len(0)
    dec.decode_streams(np.array([int(ids[-1, 0])], np.int32), args.profile_steps)
    fam = {f: dec.profile_read(f) for f in ("decode_attn", "kv_append", "projections", "logits")}
    dec.profile(False)
    attn_ms, attn_n = fam["decode_attn"]
    attn_us = attn_ms * 1e3 / attn_n
    L_avg = ctx1 + 1 + (args.profile_steps - 1) / 2.0
    attn_bytes = 4096.0 * L_avg + 16384.0
    achieved = attn_bytes / (attn_us * 1e-6) / 1e9
    log("per-step device time by family (ms): " +
        ", ".join(f"{k} {v[0] / args.profile_steps:.3f}" for k, v in fam.items()))

    result = {
        "metric": METRIC,
        "value": round(args.steps / dt, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) audio rows, random prompt ids)",
        "config": {"workload": f"config {args.config}: {w.size.name} decoder, prefill {w.prompt} positions, greedy "
                               f"decode at context {ctx0}..{ctx0 + args.steps}, f16 KV cache, f32 weights, batch 1",
                   "kv_cache": "f16", "prompt_positions": w.prompt},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode attention (decode_scores_kernel + decode_values_kernel) per layer call",
                     "bytes_per_launch": round(attn_bytes), "avg_launch_us": round(attn_us, 3)},
        "attn_us_per_layer": round(attn_us, 3),
        "prefill_ms": round(prefill_ms, 2),
        "weight_bytes_per_token": int(4 * sum(model.tensor(n).size for n in (
            [f"text.blk.{l}.{t}.weight" for l in range(model.cfg.n_layers) for t in
             ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")] + ["text.output.weight"]))),
    }
    dec.close()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(model, ctx0, args.cpu_steps)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
