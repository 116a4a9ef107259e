"""Decode benchmark of the MI355X Qwen3-ASR text decoder (BASELINE metric, one GPU).

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--config 3] [--no-cpu-baseline]

Workload (config 3): Qwen3-ASR-1.7B decoder, seeded N(0, 0.02) weights, f16 KV cache, prefill of
3913 positions (3900 audio rows + 13 random prompt ids), then greedy decode at ~4k context.  The
weights are rounded to bf16 values and kept as f32 (--weights bf16-exact, the default): a checkpoint
converted from the released bf16 weights holds exactly such values (convert.py:386-387 widens each
bf16 tensor with tensor.float()).  The decoder then streams bf16 copies of them and computes the same
f32 results; --weights f32 keeps unrounded draws (f32 weights streamed).  A short decode of the same
model with the f32 weights streamed (QA_WEIGHTS_F32=1) is reported beside the main figure.
A step is one decode token: embedding gather, 28 layers (q|k|v GEMV, fused K/V append + split-K
attention, o / gate-up / down GEMVs), LM head and device argmax.  value = decode tokens/s over exactly
--steps steps, weights and cache resident in HBM, bracketed by device synchronisation.

roofline: the decode-step attention of one layer (fused K/V append + split-K attention: the scores
and values kernels).  Its average duration per layer is measured with HIP events on the decoder's
stream around a back-to-back loop at the benchmark's context, rotating through all 28 layer caches
so the 256 MB MALL cannot serve them (470 MB of KV per token).  Algorithmic bytes per launch =
4096 * L + 16384 (K and V rows of L positions in f16, plus q in and o out in f32).

cpu_baseline: the CPU oracle (oracle/qa_oracle.c, a restatement of the reference's graph
semantics, OpenMP) decoding a bounded number of tokens of the same model at the same context.
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


def host_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return min(n, 16)   # the GPU box grants 16 host cores per GPU


def cpu_baseline(model, length: int, steps: int):
    """Oracle decode steps of the same model at the same context (cache rows N(0, 1), f16)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import qa_oracle as orc
    import qwenasr_amd as qa

    cores = host_cores()
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
    # the oracle reads every f32 weight once per token (it has no bf16 copies), plus the f16 cache prefix
    wbytes = 4 * sum(model.tensor(f"text.blk.{l}.{t}.weight").size for l in range(c.n_layers)
                     for t in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"))
    wbytes += 4 * model.tensor("text.output.weight").size
    kv = 2 * 2 * c.n_layers * c.n_kv_heads * c.head_dim * (length + steps // 2)
    gbs = (wbytes + kv) * steps / dt / 1e9
    return dict(value=round(steps / dt, 4), unit="tok/s", cores=cores, kind="port",
                sample=f"{steps} decode steps of the 1.7B decoder by the CPU oracle (C, OpenMP, {cores} threads) at "
                       f"context {length + 1}..{length + steps + 1}, f16 cache, {dt:.1f} s; it streams the f32 "
                       f"weights and the cache prefix at {gbs:.0f} GB/s of host memory")


def measured_traffic(bytes_per_launch: int):
    """HBM bytes per decode-attention launch pair from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    measurement (scaled by the plain-copy calibration), carried to this run's context by the measured
    traffic / algorithmic ratio; None when the measurement file is absent."""
    path = os.path.join(ROOT, "profiles", "decode_attention_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    ratio = t["traffic_bytes"] / t["algorithmic_bytes"]
    return round(ratio * bytes_per_launch), {"measured_at_positions": t["attended_positions"],
                                            "traffic_over_algorithmic": round(ratio, 4), "source": t["source"]}


def attention_roofline(qa, dec, reps: int):
    """Average duration of one layer's decode-step attention (fused append + split-K attention: the
    scores and values kernels), back to back on the decoder stream, HIP events from the C ABI."""
    import ctypes as C

    import numpy as np

    lay = qa.KvLayout()
    cache = qa.lib.qa_decoder_cache(dec.handle, C.byref(lay))
    s_ptr = qa.lib.qa_decoder_stream(dec.handle)
    cfg = dec.cfg
    q_dim, kv_dim = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    ctx = dec.cur_len(0)                       # the kernels append at row ctx and attend ctx + 1 rows
    assert ctx + 1 <= lay.max_seq
    qkv = qa.DeviceArray.from_numpy(np.random.default_rng(5).standard_normal((1, q_dim + 2 * kv_dim)).astype(np.float32))
    ones = qa.DeviceArray.from_numpy(np.ones(cfg.head_dim, np.float32))
    n_past = qa.DeviceArray.from_numpy(np.array([ctx], np.int32))
    out = qa.DeviceArray((1, q_dim))
    ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(lay.n_streams, cfg.n_heads, lay.max_seq)
    ws = qa.DeviceArray(ws_bytes, np.uint8)
    qa.synchronize()
    scale = 1.0 / (cfg.head_dim ** 0.5)

    def launch(layer):
        qa.check(qa.lib.qa_decode_step_attn(qkv.ptr, ones.ptr, ones.ptr, C.c_void_p(cache), C.byref(lay), layer,
                                            n_past.ptr, 1, ctx + 1, cfg.n_heads, cfg.rope_theta, cfg.rms_norm_eps,
                                            scale, out.ptr, ws.ptr, ws_bytes, C.c_void_p(s_ptr)))

    for layer in range(lay.n_layers):          # warm
        launch(layer)
    e0, e1 = C.c_void_p(), C.c_void_p()
    qa.check(qa.lib.qa_event_create(C.byref(e0)))
    qa.check(qa.lib.qa_event_create(C.byref(e1)))
    qa.check(qa.lib.qa_event_record(e0, C.c_void_p(s_ptr)))
    for _ in range(reps):
        for layer in range(lay.n_layers):
            launch(layer)
    qa.check(qa.lib.qa_event_record(e1, C.c_void_p(s_ptr)))
    ms = C.c_float()
    qa.check(qa.lib.qa_event_elapsed_ms(e0, e1, C.byref(ms)))
    qa.lib.qa_event_destroy(e0)
    qa.lib.qa_event_destroy(e1)
    n = reps * lay.n_layers
    us = ms.value * 1e3 / n
    L = ctx + 1
    elem = 2 if lay.cache_type == qa.QA_CACHE_F16 else 4
    bytes_per_launch = 2 * cfg.n_kv_heads * cfg.head_dim * elem * L + 16384   # K and V rows, q in, o out
    return us, L, bytes_per_launch, n


def copy_calibration(reps: int = 10, mib: int = 256):
    """A plain device-to-device copy of known size: the reference that rocprofv3's FETCH_SIZE and
    WRITE_SIZE counters (KiB per dispatch) are scaled by when they are turned into HBM bytes."""
    import numpy as np
    import qwenasr_amd as qa

    n = mib << 20
    src = qa.DeviceArray(n, np.uint8)
    dst = qa.DeviceArray(n, np.uint8, zero=False)
    qa.synchronize()
    for _ in range(reps):
        qa.check(qa.lib.qa_copy_device(dst.ptr, src.ptr, n, None))
    qa.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_per_copy": n, "copies": reps}}), flush=True)


def multistream_roofline(qa, cfg, reps: int, lens=None, label: str = "config 4 shapes"):
    """Multi-stream decode-step attention: one launch pair per layer covering every stream, rotating over
    28 layer caches (so no cache can serve them).  Default lengths: config 4's seeded U[156, 3913]
    (14.6 GB of f16 KV).  Cache contents do not change the bytes moved, so the cache stays zeroed."""
    import ctypes as C

    import numpy as np
    from qwenasr_amd import configs

    if lens is None:
        lens = configs.cfg4_lengths(configs.CONFIGS[4].streams)
    lens = np.asarray(lens).astype(np.int32)
    S = len(lens)
    cap = int(lens.max()) + 2
    lay = qa.KvLayout(cfg.n_layers, S, cfg.n_kv_heads, cfg.head_dim, cap, qa.QA_CACHE_F16)
    cache = qa.DeviceArray(qa.lib.qa_kv_cache_bytes(C.byref(lay)), np.uint8)
    q_dim, kv_dim = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    qkv = qa.DeviceArray.from_numpy(np.random.default_rng(6).standard_normal((S, q_dim + 2 * kv_dim)).astype(np.float32))
    ones = qa.DeviceArray.from_numpy(np.ones(cfg.head_dim, np.float32))
    n_past = qa.DeviceArray.from_numpy(lens)
    out = qa.DeviceArray((S, q_dim))
    ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(S, cfg.n_heads, cap)
    ws = qa.DeviceArray(ws_bytes, np.uint8)
    qa.synchronize()
    scale = 1.0 / (cfg.head_dim ** 0.5)
    max_len = int(lens.max()) + 1

    def launch(layer):
        qa.check(qa.lib.qa_decode_step_attn(qkv.ptr, ones.ptr, ones.ptr, cache.ptr, C.byref(lay), layer, n_past.ptr, S,
                                            max_len, cfg.n_heads, cfg.rope_theta, cfg.rms_norm_eps, scale, out.ptr,
                                            ws.ptr, ws_bytes, None))

    for layer in range(lay.n_layers):
        launch(layer)
    e0, e1 = C.c_void_p(), C.c_void_p()
    qa.check(qa.lib.qa_event_create(C.byref(e0)))
    qa.check(qa.lib.qa_event_create(C.byref(e1)))
    qa.check(qa.lib.qa_event_record(e0, None))
    for _ in range(reps):
        for layer in range(lay.n_layers):
            launch(layer)
    qa.check(qa.lib.qa_event_record(e1, None))
    ms = C.c_float()
    qa.check(qa.lib.qa_event_elapsed_ms(e0, e1, C.byref(ms)))
    qa.lib.qa_event_destroy(e0)
    qa.lib.qa_event_destroy(e1)
    us = ms.value * 1e3 / (reps * lay.n_layers)
    nbytes = int(sum(4096 * (int(L) + 1) + 16384 for L in lens))
    achieved = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "bytes_per_launch": nbytes, "avg_launch_us": round(us, 3),
            "workload": f"{label}: {S} streams, contexts {int(lens.min()) + 1}..{int(lens.max()) + 1} "
                        f"(mean {float(lens.mean()) + 1:.0f}), one layer's decode-step attention per launch pair"}


def kernel_only(which: str, reps: int):
    """One hot-path kernel on synthetic inputs at the config-3 shape, for rocprofv3 passes (the counters
    of every dispatch are then the kernel's alone).  append: the prefill K/V append of 3913 positions
    (q/k norm + RoPE, f16 cache write); prefill: causal prefill attention over 3913 positions of one
    layer (f16 cache, n_past 0); decode-attn: the decode-step attention of one layer at L = 4186,
    rotating 28 layer caches; multistream: the config-4 decode step of 32 streams (end to end);
    multistream-attn: the decode-step attention of 32 streams at L = 4096 (reps x 28 launch pairs)."""
    if which == "multistream-attn":
        import qwenasr_amd as qa

        cfg = qa.QWEN3_ASR_1_7B.config()
        r = multistream_roofline(qa, cfg, reps, lens=[4095] * 32, label="32 streams at 4k context")
        print(json.dumps(dict(kernel=which, **r)), flush=True)
        return
    if which == "multistream":
        import qwenasr_amd as qa
        from qwenasr_amd import configs

        w = configs.CONFIGS[4]
        model = qa.Model(w.size, n_layers=w.n_layers, bf16=True)
        print(json.dumps(dict(kernel=which, **multistream_decode(qa, model, reps))), flush=True)
        return
    import ctypes as C

    import numpy as np
    import qwenasr_amd as qa

    cfg = qa.QWEN3_ASR_1_7B.config()
    scale = 1.0 / (cfg.head_dim ** 0.5)
    e0, e1 = C.c_void_p(), C.c_void_p()
    qa.check(qa.lib.qa_event_create(C.byref(e0)))
    qa.check(qa.lib.qa_event_create(C.byref(e1)))
    if which == "append":
        T = 3913
        lay = qa.KvLayout(2, 1, cfg.n_kv_heads, cfg.head_dim, T + 8, qa.QA_CACHE_F16)
        cache = qa.DeviceArray(qa.lib.qa_kv_cache_bytes(C.byref(lay)), np.uint8)
        q_dim, kv_dim = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        qkv = qa.DeviceArray.from_numpy(np.random.default_rng(4).standard_normal((T, q_dim + 2 * kv_dim)).astype(np.float32))
        ones = qa.DeviceArray.from_numpy(np.ones(cfg.head_dim, np.float32))
        q_out = qa.DeviceArray((T, q_dim))
        n_past = qa.DeviceArray.from_numpy(np.zeros(1, np.int32))

        def launch(i):
            qa.check(qa.lib.qa_kv_append(qkv.ptr, ones.ptr, ones.ptr, q_out.ptr, cache.ptr, C.byref(lay), i % 2,
                                         n_past.ptr, 1, T, cfg.n_heads, cfg.rope_theta, cfg.rms_norm_eps, None))
        # read q|k|v rows (f32), write q (f32) and the K and V rows (f16)
        unit = dict(algorithmic_bytes_per_launch=T * ((q_dim + 2 * kv_dim) * 4 + q_dim * 4 + 2 * kv_dim * 2))
    elif which == "prefill":
        T = 3913
        lay = qa.KvLayout(2, 1, cfg.n_kv_heads, cfg.head_dim, T + 8, qa.QA_CACHE_F16)
        cache = qa.DeviceArray(qa.lib.qa_kv_cache_bytes(C.byref(lay)), np.uint8)
        q = qa.DeviceArray.from_numpy(np.random.default_rng(3).standard_normal((T, cfg.n_heads * cfg.head_dim)).astype(np.float32))
        out = qa.DeviceArray((T, cfg.n_heads * cfg.head_dim))
        wsb = qa.lib.qa_prefill_attn_workspace_bytes(T, cfg.n_heads)
        ws = qa.DeviceArray(max(wsb, 256), np.uint8)

        def launch(i):
            qa.check(qa.lib.qa_prefill_attn(q.ptr, cache.ptr, C.byref(lay), i % 2, 0, 0, T, cfg.n_heads, scale, out.ptr,
                                            ws.ptr, wsb, None))
        flops = 4.0 * cfg.n_heads * cfg.head_dim * T * (T + 1) / 2
        unit = dict(useful_gflop_per_launch=round(flops / 1e9, 3))
    else:
        L = 4186
        lay = qa.KvLayout(cfg.n_layers, 1, cfg.n_kv_heads, cfg.head_dim, L + 8, qa.QA_CACHE_F16)
        cache = qa.DeviceArray(qa.lib.qa_kv_cache_bytes(C.byref(lay)), np.uint8)
        q_dim, kv_dim = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        qkv = qa.DeviceArray.from_numpy(np.random.default_rng(5).standard_normal((1, q_dim + 2 * kv_dim)).astype(np.float32))
        ones = qa.DeviceArray.from_numpy(np.ones(cfg.head_dim, np.float32))
        n_past = qa.DeviceArray.from_numpy(np.array([L - 1], np.int32))
        out = qa.DeviceArray((1, q_dim))
        wsb = qa.lib.qa_decode_attn_workspace_bytes(1, cfg.n_heads, lay.max_seq)
        ws = qa.DeviceArray(wsb, np.uint8)

        def launch(i):
            qa.check(qa.lib.qa_decode_step_attn(qkv.ptr, ones.ptr, ones.ptr, cache.ptr, C.byref(lay), i % cfg.n_layers,
                                                n_past.ptr, 1, L, cfg.n_heads, cfg.rope_theta, cfg.rms_norm_eps, scale,
                                                out.ptr, ws.ptr, wsb, None))
        unit = dict(algorithmic_bytes_per_launch=4096 * L + 16384)
    launch(0)
    qa.synchronize()
    qa.check(qa.lib.qa_event_record(e0, None))
    for i in range(reps):
        launch(i)
    qa.check(qa.lib.qa_event_record(e1, None))
    ms = C.c_float()
    qa.check(qa.lib.qa_event_elapsed_ms(e0, e1, C.byref(ms)))
    us = ms.value * 1e3 / reps
    print(json.dumps(dict(kernel=which, launches=reps + 1, avg_us=round(us, 3), **unit)), flush=True)


def multistream_decode(qa, model, steps: int):
    """Config 4 end to end: 32 streams at the config's seeded ragged lengths (156..3913), lock-step
    greedy decode (per step: embedding, 28 layers with f32 projections of 32 rows, fused append +
    split-K attention over every stream, LM head, argmax).  Cache contents do not change the time, so
    the lengths are set without filling K/V.  value = aggregate generated tokens per second."""
    import numpy as np
    from qwenasr_amd import configs

    w = configs.CONFIGS[4]
    lens = configs.cfg4_lengths(w.streams)
    first = configs.cfg4_first_ids(w.streams).astype(np.int32)
    with qa.Decoder(model, w.streams, w.max_seq, w.cache_type) as dec:
        streamed = "bf16 copies of bf16-exact weights" if dec.weights_bf16 else "f32 weights"
        for s_ in range(w.streams):
            dec.set_cur_len(s_, int(lens[s_]))
        ids = dec.decode_streams(first, 2)                  # warm
        bad = [(k, s_, int(ids[k, s_])) for k in range(ids.shape[0]) for s_ in range(ids.shape[1])
               if not 0 <= int(ids[k, s_]) < model.cfg.vocab]
        assert not bad, f"config-4 warm-up produced invalid ids (step, stream, id): {bad[:8]}"
        qa.check(qa.lib.qa_device_synchronize())
        t0 = time.perf_counter()
        last = dec.decode_streams(ids[-1].astype(np.int32), steps)
        qa.check(qa.lib.qa_device_synchronize())
        dt = time.perf_counter() - t0
        # where a step's device time goes (HIP events around each kernel family, outside the timed steps)
        n_prof = 4
        dec.profile(True)
        dec.profile_reset()
        dec.decode_streams(last[-1].astype(np.int32), n_prof)
        fam = {f: round(dec.profile_read(f)[0] / n_prof, 3) for f in ("decode_attn", "projections", "logits")}
        dec.profile(False)
    return {"streams": w.streams, "steps": steps, "ms_per_step": round(dt * 1e3 / steps, 3),
            "tok_s": round(w.streams * steps / dt, 1), "family_ms_per_step": fam,
            "workload": f"config 4: {w.streams} streams, contexts {int(lens.min())}..{int(lens.max())} + {steps + 2}, "
                        f"lock-step greedy decode, f16 cache, {streamed} streamed"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", type=int, default=3, choices=[2, 3])
    ap.add_argument("--roofline-reps", type=int, default=20)
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--multistream-steps", type=int, default=16)
    ap.add_argument("--cpu-steps", type=int, default=192, help="oracle decode steps of the CPU baseline (~10-20 s)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--weights", choices=["bf16-exact", "f32"], default="bf16-exact",
                    help="bf16-exact: weights rounded to bf16 values (a converted bf16 checkpoint); f32: unrounded")
    ap.add_argument("--kv-cache", choices=["f16", "f32"], default=None,
                    help="cache type (default: the config's, f16 for configs 2 and 3; f32 is the drop-in's default)")
    ap.add_argument("--f32-compare-steps", type=int, default=64,
                    help="decode steps timed with the f32 weights streamed, on the same model (0: skip)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy 10 times (reference for HBM traffic counters)")
    ap.add_argument("--kernel", choices=["append", "prefill", "decode-attn", "multistream", "multistream-attn"],
                    help="only run one hot-path kernel on synthetic inputs (short program for rocprofv3 passes)")
    ap.add_argument("--kernel-reps", type=int, default=20)
    args = ap.parse_args()
    if args.kernel:
        kernel_only(args.kernel, args.kernel_reps)
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the KV-cache path would shard by "
              "KV head or by stream); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import qwenasr_amd as qa
    from qwenasr_amd import configs

    assert qa.device_count() > 0, "bench.py needs a HIP device"
    w = configs.CONFIGS[args.config]
    t0 = time.perf_counter()
    model = qa.Model(w.size, n_layers=w.n_layers, bf16=args.weights == "bf16-exact")
    x = qa.prompt_input(model, w.audio_tokens, w.prompt_tokens)
    log(f"synthetic {w.size.name} ({args.weights} weights) built in {time.perf_counter() - t0:.1f}s")
    max_seq = w.prompt + args.warmup + args.steps + args.profile_steps + 2
    if args.kv_cache:
        import dataclasses
        w = dataclasses.replace(w, cache_type=qa.QA_CACHE_F16 if args.kv_cache == "f16" else qa.QA_CACHE_F32)
    kv_name = "f16" if w.cache_type == qa.QA_CACHE_F16 else "f32"
    dec = qa.Decoder(model, 1, max_seq, w.cache_type)
    weights_streamed = "bf16 copies of bf16-exact weights" if dec.weights_bf16 else "f32"
    log(f"decoder ready (weights + {max_seq}-position {kv_name} cache on device; GEMVs stream {weights_streamed})")

    # the first prefill also allocates the prompt-sized workspaces and loads rocBLAS's kernels; the
    # second (same input, n_past 0 again: the cache rows are rewritten) is the steady-state time
    qa.check(qa.lib.qa_device_synchronize())
    t0 = time.perf_counter()
    logits = dec.forward(x, 0)
    prefill_cold_ms = (time.perf_counter() - t0) * 1e3
    t0 = time.perf_counter()
    logits = dec.forward(x, 0)
    prefill_ms = (time.perf_counter() - t0) * 1e3
    first = int(np.argmax(logits))
    # a third, event-bracketed prefill for the split by kernel family (events add gaps: upper bounds)
    dec.profile(True)
    dec.profile_reset()
    dec.forward(x, 0, want_logits=False)
    prefill_fam = {f: round(dec.profile_read(f)[0], 2) for f in ("projections", "kv_append", "prefill_attn", "logits")}
    dec.profile(False)
    log(f"prefill {w.prompt} positions: {prefill_ms:.1f} ms (first call {prefill_cold_ms:.1f} ms); "
        f"device ms by family {prefill_fam}")

    ids = dec.decode_streams(np.array([first], np.int32), args.warmup) if args.warmup else np.array([[first]])
    last = int(ids[-1, 0])
    qa.check(qa.lib.qa_device_synchronize())
    ctx0 = dec.cur_len(0)
    t0 = time.perf_counter()
    ids = dec.decode_streams(np.array([last], np.int32), args.steps)
    qa.check(qa.lib.qa_device_synchronize())
    dt = time.perf_counter() - t0
    log(f"timed {args.steps} decode steps at context {ctx0}..{ctx0 + args.steps}: {dt * 1e3:.1f} ms "
        f"({dt * 1e3 / args.steps:.3f} ms/token)")

    # per-step device time by kernel family (HIP events around each family; events add gaps, so these
    # are upper bounds used only for the breakdown)
    dec.profile(True)
    dec.profile_reset()
    dec.decode_streams(np.array([int(ids[-1, 0])], np.int32), args.profile_steps)
    fam = {f: dec.profile_read(f) for f in ("decode_attn", "projections", "logits")}
    dec.profile(False)
    log("per-step device time by family, event-bracketed (ms): " +
        ", ".join(f"{k} {v[0] / args.profile_steps:.3f}" for k, v in fam.items()))

    f32_cmp = None
    if args.f32_compare_steps > 0 and dec.weights_bf16:
        # the same model and context with the f32 weights streamed (the kernels the golden tests pin)
        os.environ["QA_WEIGHTS_F32"] = "1"
        d32 = qa.Decoder(model, 1, max_seq, w.cache_type)
        del os.environ["QA_WEIGHTS_F32"]
        d32.forward(x, 0, want_logits=False)
        warm = d32.decode_streams(np.array([first], np.int32), args.warmup) if args.warmup else np.array([[first]])
        qa.check(qa.lib.qa_device_synchronize())
        t1 = time.perf_counter()
        ids32 = d32.decode_streams(np.array([int(warm[-1, 0])], np.int32), args.f32_compare_steps)
        qa.check(qa.lib.qa_device_synchronize())
        dt32 = time.perf_counter() - t1
        d32.close()
        # the same arithmetic on the same values: the ids follow the main run's token for token
        n_cmp = min(args.f32_compare_steps, args.steps)
        same = bool(np.array_equal(ids32[:n_cmp, 0], ids[:n_cmp, 0]))
        f32_cmp = {"steps": args.f32_compare_steps, "ms_per_step": round(dt32 * 1e3 / args.f32_compare_steps, 4),
                   "tok_s": round(args.f32_compare_steps / dt32, 3), "ids_equal_to_main_run": same,
                   "weight_bytes_per_token": None}
        log(f"same model, f32 weights streamed: {f32_cmp['ms_per_step']:.3f} ms/token (ids equal: {same})")

    attn_us, L, attn_bytes, n_launch = attention_roofline(qa, dec, args.roofline_reps)
    achieved = attn_bytes / (attn_us * 1e-6) / 1e9
    log(f"decode-step attention: {attn_us:.2f} us per launch over {n_launch} launches at L={L}: "
        f"{achieved:.0f} GB/s")

    dec.close()
    roof4 = multistream_roofline(qa, model.cfg, max(2, args.roofline_reps // 4))
    log(f"config-4 multi-stream attention: {roof4['avg_launch_us']:.1f} us per layer, {roof4['achieved']:.0f} GB/s "
        f"({100 * roof4['frac']:.1f}% of peak)")

    roof4k = multistream_roofline(qa, model.cfg, max(2, args.roofline_reps // 4), lens=[4095] * 32,
                                  label="32 streams at 4k context")
    log(f"32 streams at 4k: {roof4k['avg_launch_us']:.1f} us per layer, {roof4k['achieved']:.0f} GB/s "
        f"({100 * roof4k['frac']:.1f}% of peak)")
    ms4 = multistream_decode(qa, model, args.multistream_steps)
    log(f"config-4 decode, {ms4['streams']} streams: {ms4['ms_per_step']:.2f} ms per step, {ms4['tok_s']:.0f} tok/s "
        f"(device ms per step by family: {ms4['family_ms_per_step']})")

    traffic, traffic_note = measured_traffic(attn_bytes)
    n_weights = int(sum(model.tensor(n).size for n in (
        [f"text.blk.{l}.{t}.weight" for l in range(model.cfg.n_layers) for t in
         ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")] + ["text.output.weight"])))
    weight_bytes = n_weights * (2 if weights_streamed != "f32" else 4)
    if f32_cmp is not None:
        f32_cmp["weight_bytes_per_token"] = 4 * n_weights
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
        "data": (f"synthetic (seeded N(0,0.02) weights{', rounded to bf16 values as in a converted bf16 checkpoint' if args.weights == 'bf16-exact' else ''}, "
                 f"N(0,1) audio rows, random prompt ids)"),
        "config": {"workload": f"config {args.config}: {w.size.name} decoder, prefill {w.prompt} positions, greedy "
                               f"decode of {args.steps} tokens at context {ctx0}..{ctx0 + args.steps}, {kv_name} KV cache, "
                               f"{args.weights} weights, batch 1",
                   "kv_cache": kv_name, "prompt_positions": w.prompt, "weights": args.weights,
                   "weights_streamed": weights_streamed},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": traffic_note,
                     "kernel": "decode attention of one layer: decode_scores_kernel (fused K/V append) + "
                               "decode_values_kernel, launched back to back",
                     "bytes_per_launch": attn_bytes, "attended_positions": L, "avg_launch_us": round(attn_us, 3)},
        "roofline_multistream": roof4,
        "roofline_multistream_4k": roof4k,
        "multistream_decode": ms4,
        "attn_us_per_layer": round(attn_us, 3),
        "prefill_ms": round(prefill_ms, 2),
        "prefill_first_call_ms": round(prefill_cold_ms, 2),
        "prefill_family_ms": prefill_fam,
        "weight_bytes_per_token": weight_bytes,
        "weight_stream_gbs": round(weight_bytes / (dt / args.steps) / 1e9, 1),
        "decode_f32_weights_streamed": f32_cmp,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(model, ctx0, args.cpu_steps)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
