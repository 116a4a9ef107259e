"""Decode benchmark of the MI355X Qwen3-ASR text decoder (BASELINE metric, one GPU).

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--config 3] [--no-cpu-baseline]

Workload (config 3): Qwen3-ASR-1.7B decoder, seeded N(0, 0.02) weights streamed as
f32 (the reference's contract: every weight an f32 tensor, require_f32_tensor text-decoder.cpp:29-42),
f16 KV cache, prefill of 3913 positions (3900 audio rows + 13 random prompt ids), then greedy decode at
~4k context, batch 1.  A step is one decode token: embedding gather, 28 layers (q|k|v GEMV, fused K/V
append + split-K attention, o / gate-up / down GEMVs), LM head and device argmax.  value = decode
tokens/s over exactly --steps steps, weights and cache resident in HBM, bracketed by device
synchronisation.

Each decoder is sized for the legs it runs (capacity_plan).  The secondary legs record an "error"
object instead of ending the run: the f32-cache attention roofline, the config-4 (32-stream)
attention and decode step, the CPU baseline, and the same draws rounded to bf16 values
(decode_bf16_exact_weights: what a checkpoint converted from the released bf16 weights holds,
convert.py:386-387; the decoder then streams bf16 copies of them, with f32 products and sums).

roofline: the decode-step attention of one layer (fused K/V append + split-K attention: the scores
and values kernels).  Its average duration per layer is measured with HIP events on the decoder's
stream around a back-to-back loop at the benchmark's context, rotating through all 28 layer caches
so the 256 MB MALL cannot serve them (470 MB of KV per token).  Algorithmic bytes per launch =
4096 * L + 16384 (K and V rows of L positions in f16, plus q in and o out in f32); 8192 * L + 16384
for the f32 cache (roofline_f32_cache).

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
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense f16 / bf16 MFMA, MI355X


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


def measured_traffic(bytes_per_launch: int, kv_name: str = "f16"):
    """HBM bytes per decode-attention launch pair from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    measurement of that cache type (scaled by the plain-copy calibration), carried to this run's context
    by the measured traffic / algorithmic ratio; None when the measurement file is absent."""
    name = "decode_attention_traffic.json" if kv_name == "f16" else f"decode_attention_traffic_{kv_name}.json"
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    ratio = t["traffic_bytes"] / t["algorithmic_bytes"]
    return round(ratio * bytes_per_launch), {"measured_at_positions": t["attended_positions"],
                                            "traffic_over_algorithmic": round(ratio, 4), "source": t["source"]}


def f32_cache_roofline(qa, cfg, L: int, reps: int):
    """Batch-1 decode-step attention over an f32 cache (the reference's cache dtype, text-decoder.cpp:
    1451-1462, and the drop-in's default) at L attended positions, rotating 28 layer caches; algorithmic
    bytes per launch pair = 8192 * L + 16384 (f32 K and V rows, q in, o out)."""
    us = attn_pair_us(qa, cfg, L, qa.QA_CACHE_F32, reps)
    nbytes = 8192 * L + 16384
    achieved = nbytes / (us * 1e-6) / 1e9
    traffic, note = measured_traffic(nbytes, "f32")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": note,
            "bytes_per_launch": nbytes, "attended_positions": L, "avg_launch_us": round(us, 3),
            "kernel": "decode_scores_kernel (fused K/V append) + decode_values_kernel, f32 cache"}


def attn_pair_us(qa, cfg, L: int, cache_type: int, reps: int) -> float:
    """Average microseconds of one batch-1 qa_decode_step_attn call at L attended positions (append at
    row L - 1), back to back over reps x 28 launches rotating the layer caches, HIP events on the null
    stream.  The cache holds zeros: its contents do not change the bytes moved."""
    import ctypes as C

    import numpy as np

    lay = qa.KvLayout(cfg.n_layers, 1, cfg.n_kv_heads, cfg.head_dim, L + 8, cache_type)
    cache = qa.DeviceArray(qa.lib.qa_kv_cache_bytes(C.byref(lay)), np.uint8)
    q_dim, kv_dim = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    qkv = qa.DeviceArray.from_numpy(np.random.default_rng(5).standard_normal((1, q_dim + 2 * kv_dim)).astype(np.float32))
    ones = qa.DeviceArray.from_numpy(np.ones(cfg.head_dim, np.float32))
    n_past = qa.DeviceArray.from_numpy(np.array([L - 1], np.int32))
    out = qa.DeviceArray((1, q_dim))
    wsb = qa.lib.qa_decode_attn_workspace_bytes(1, cfg.n_heads, lay.max_seq)
    ws = qa.DeviceArray(wsb, np.uint8)
    scale = 1.0 / (cfg.head_dim ** 0.5)

    def launch(layer):
        qa.check(qa.lib.qa_decode_step_attn(qkv.ptr, ones.ptr, ones.ptr, cache.ptr, C.byref(lay), layer, n_past.ptr, 1,
                                            L, cfg.n_heads, cfg.rope_theta, cfg.rms_norm_eps, scale, out.ptr, ws.ptr,
                                            wsb, None))

    for layer in range(cfg.n_layers):
        launch(layer)
    qa.synchronize()
    e0, e1 = C.c_void_p(), C.c_void_p()
    qa.check(qa.lib.qa_event_create(C.byref(e0)))
    qa.check(qa.lib.qa_event_create(C.byref(e1)))
    qa.check(qa.lib.qa_event_record(e0, None))
    for _ in range(reps):
        for layer in range(cfg.n_layers):
            launch(layer)
    qa.check(qa.lib.qa_event_record(e1, None))
    ms = C.c_float()
    qa.check(qa.lib.qa_event_elapsed_ms(e0, e1, C.byref(ms)))
    qa.lib.qa_event_destroy(e0)
    qa.lib.qa_event_destroy(e1)
    return ms.value * 1e3 / (reps * cfg.n_layers)


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


def kernel_only(which: str, reps: int, weights: str = "f32", length: int = 4186):
    """One hot-path kernel on synthetic inputs at the config-3 shape, for rocprofv3 passes (the counters
    of every dispatch are then the kernel's alone).  append: the prefill K/V append of 3913 positions
    (q/k norm + RoPE, f16 cache write); prefill / prefill-f32: causal prefill attention over 3913 positions
    of one layer (f16 / f32 cache, n_past 0); decode-attn / decode-attn-f32: the decode-step attention of one layer
    at L = length (default 4186, capacity L + 8) over an f16 / f32 cache, rotating 28 layer caches; decode-step: config 3 end to end at
    batch 1 (prefill once, then reps greedy decode tokens), decode-step-persistent the same with every
    layer of a token in one persistent launch; multistream: the config-4 decode step of 32
    streams (end to end); multistream-attn: the decode-step attention of 32 streams at L = 4096 (reps x
    28 launch pairs).  weights: f32 or bf16-exact draws for the end-to-end modes."""
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
        model = qa.Model(w.size, n_layers=w.n_layers, bf16=weights == "bf16-exact")
        print(json.dumps(dict(kernel=which, weights=weights, **multistream_decode(qa, model, reps))), flush=True)
        return
    if which in ("decode-step", "decode-step-persistent"):
        import numpy as np
        import qwenasr_amd as qa
        from qwenasr_amd import configs

        w = configs.CONFIGS[3]
        model = qa.Model(w.size, n_layers=w.n_layers, bf16=weights == "bf16-exact")
        x = qa.prompt_input(model, w.audio_tokens, w.prompt_tokens)
        with qa.Decoder(model, 1, w.prompt + reps + 8, w.cache_type) as dec:
            if which == "decode-step-persistent":
                dec.set_persistent(True)
            logits = dec.forward(x, 0)
            ids = dec.decode_streams(np.array([int(np.argmax(logits))], np.int32), 2)
            qa.synchronize()
            t0 = time.perf_counter()
            dec.decode_streams(np.array([int(ids[-1, 0])], np.int32), reps)
            qa.synchronize()
            dt = time.perf_counter() - t0
            streamed = "bf16 copies" if dec.weights_bf16 else "f32"
        print(json.dumps(dict(kernel=which, weights=weights, weights_streamed=streamed, steps=reps,
                              ms_per_step=round(dt * 1e3 / reps, 4))), flush=True)
        return
    if which == "decode-attn-f32":
        import qwenasr_amd as qa

        cfg = qa.QWEN3_ASR_1_7B.config()
        L = length
        us = attn_pair_us(qa, cfg, L, qa.QA_CACHE_F32, max(1, reps // cfg.n_layers))
        print(json.dumps(dict(kernel=which, avg_us=round(us, 3), algorithmic_bytes_per_launch=8192 * L + 16384)),
              flush=True)
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
    elif which in ("prefill", "prefill-f32"):
        T = 3913
        ct = qa.QA_CACHE_F16 if which == "prefill" else qa.QA_CACHE_F32
        lay = qa.KvLayout(2, 1, cfg.n_kv_heads, cfg.head_dim, T + 8, ct)
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
        L = length
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


def capacity_plan(prompt: int, warmup: int, steps: int, profile_steps: int, bf16_steps: int,
                  persistent_steps: int = 0) -> dict:
    """KV-cache capacity (positions per stream) of each decoder the bench creates, sized for the legs
    that decoder runs.  main: the prefill, the warm-up and timed decode steps, the event-bracketed
    profile steps, and the attention roofline, which appends at the context the decode left (row ctx)
    and attends ctx + 1 positions.  bf16_exact: its own prefill, warm-up and timed steps; persistent: the
    same for the persistent decode step.  One spare position each, so a step count of zero still leaves
    the roofline a row to append."""
    if min(prompt, warmup, steps, profile_steps, bf16_steps, persistent_steps) < 0 or prompt < 1:
        raise ValueError("capacity_plan: counts must be non-negative and the prompt non-empty")
    return {"main": prompt + warmup + steps + profile_steps + 2,
            "bf16_exact": prompt + warmup + bf16_steps + 2,
            "persistent": prompt + warmup + persistent_steps + 2}


def prefill_attn_roofline(cfg, T: int, fam_ms: dict):
    """Causal prefill attention on f16 MFMA from the prefill's event-bracketed family time: useful FLOPs
    4 n_heads head_dim T (T + 1) / 2 per layer (QK^T and PV over the unmasked half)."""
    flop = 4.0 * cfg.n_heads * cfg.head_dim * T * (T + 1) / 2 * cfg.n_layers
    ms = fam_ms["prefill_attn"]
    tf = flop / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": "prefill_mfma_kernel (f16 MFMA, single pass), all layers of one prefill",
            "flop_per_layer": round(flop / cfg.n_layers), "positions": T, "ms": ms}


def prefill_gemm_roofline(cfg, T: int, fam_ms: dict):
    """The bf16-exact prefill projections (gemm_split3: bf16 MFMA over the three-part split of each input, so
    3 x 2 T params FLOPs of MFMA work per layer) from the projection family's time, which also holds the
    RMSNorm and split passes: a lower bound on the GEMM's own rate."""
    H, QD, KD, I = cfg.hidden, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.intermediate
    params = (QD + 2 * KD) * H + H * QD + 2 * I * H + H * I
    flop = 3.0 * 2.0 * T * params * cfg.n_layers
    ms = fam_ms["projections"]
    tf = flop / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": "gemm_split3_kernel (bf16 MFMA over the split input, SwiGLU fused), the prefill's projection "
                      "family (with its RMSNorm and split passes)", "flop_per_layer": round(flop / cfg.n_layers),
            "positions": T, "ms": ms}


def decode_weight_rooflines(cfg, elem: int, fam_ms: dict):
    """HBM rooflines of the batch-1 decode step's weight streams, from the event-bracketed kernel families of
    one token (the families include the gaps between their launches, so the rates are lower bounds):
    projections = the q|k|v, o, gate|up and down GEMVs of every layer (elem bytes per parameter), lm_head = the
    final RMSNorm + LM head GEMV + greedy pick (vocab x hidden parameters)."""
    H, QD, KD, I = cfg.hidden, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.intermediate
    layer = (QD + 2 * KD) * H + H * QD + 2 * I * H + H * I
    out = {}
    for key, fam, nbytes, kernel in (
            ("projections", "projections", elem * layer * cfg.n_layers,
             "gemv_kernel: q|k|v (RMSNorm input), o (+ residual), gate|up (RMSNorm input, SwiGLU), down (+ residual), "
             "every layer of one token"),
            ("lm_head", "logits", elem * cfg.vocab * H, "gemv_kernel: final RMSNorm + LM head, then argmax_kernel")):
        ms = fam_ms[fam]
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[key] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kernel,
                    "bytes_per_token": nbytes, "ms_per_token": ms}
    return out


def guarded(result: dict, key: str, fn):
    """Runs one secondary leg; a failure is recorded under result[key] = {"error": ...} instead of ending
    the run, so the measurements taken before it still reach the JSON line."""
    try:
        result[key] = fn()
    except Exception as e:   # noqa: BLE001 - any failure of a secondary leg is reported, not raised
        log(f"{key}: {type(e).__name__}: {e}")
        result[key] = {"error": f"{type(e).__name__}: {e}"}
    return result[key]


def decode_leg(qa, model, x, cache_type, capacity: int, warmup: int, steps: int, profile_steps: int):
    """Prefill the prompt twice (cold, then steady state), warm up, time `steps` greedy decode tokens and
    split `profile_steps` more by kernel family.  Returns (decoder, figures); the caller closes it."""
    import numpy as np

    dec = qa.Decoder(model, 1, capacity, cache_type)
    # the first prefill also allocates the prompt-sized workspaces and loads the GEMM libraries' kernels;
    # the second (same input, n_past 0 again: the cache rows are rewritten) is the steady-state time
    qa.check(qa.lib.qa_device_synchronize())
    t0 = time.perf_counter()
    dec.forward(x, 0, want_logits=False)
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
    ids = dec.decode_streams(np.array([first], np.int32), warmup) if warmup else np.array([[first]], np.int32)
    all_ids = ids[:, 0].tolist() if warmup else []
    qa.check(qa.lib.qa_device_synchronize())
    ctx0 = dec.cur_len(0)
    t0 = time.perf_counter()
    ids = dec.decode_streams(np.array([int(ids[-1, 0])], np.int32), steps)
    qa.check(qa.lib.qa_device_synchronize())
    dt = time.perf_counter() - t0
    all_ids += ids[:, 0].tolist()
    fam = None
    if profile_steps > 0:
        # per-step device time by kernel family (HIP events around each family; events add gaps, so these
        # are upper bounds used only for the breakdown)
        dec.profile(True)
        dec.profile_reset()
        dec.decode_streams(np.array([int(ids[-1, 0])], np.int32), profile_steps)
        fam = {f: round(dec.profile_read(f)[0] / profile_steps, 4) for f in ("decode_attn", "projections", "logits")}
        dec.profile(False)
    return dec, {"steps": steps, "seconds": dt, "ctx0": ctx0, "ms_per_step": round(dt * 1e3 / steps, 4),
                 "tok_s": round(steps / dt, 3), "prefill_ms": round(prefill_ms, 2),
                 "prefill_first_call_ms": round(prefill_cold_ms, 2), "prefill_family_ms": prefill_fam,
                 "family_ms_per_step": fam, "first_id": first, "ids": all_ids}


def weight_bytes(model, elem: int) -> int:
    """Projection and LM-head weight bytes one decode token streams (elem: 4 for f32, 2 for bf16 copies)."""
    c = model.cfg
    n = sum(model.tensor(f"text.blk.{l}.{t}.weight").size for l in range(c.n_layers)
            for t in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"))
    return int(elem * (n + model.tensor("text.output.weight").size))


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
    ap.add_argument("--weights", choices=["f32", "bf16-exact"], default="f32",
                    help="f32: the seeded N(0, 0.02) draws as BASELINE states them (f32 weights streamed); "
                         "bf16-exact: the same draws rounded to bf16 values (a converted bf16 checkpoint)")
    ap.add_argument("--kv-cache", choices=["f16", "f32"], default=None,
                    help="cache type (default: the config's, f16 for configs 2 and 3; f32 is the drop-in's default)")
    ap.add_argument("--bf16-steps", type=int, default=64,
                    help="decode steps timed on the same draws rounded to bf16 values, whose bf16 copies the "
                         "decoder streams (a secondary object of the line; 0: skip)")
    ap.add_argument("--persistent-steps", type=int, default=32,
                    help="decode steps timed with the persistent decode step (qa_decoder_set_persistent: every "
                         "layer of a token in one launch), a secondary object of the line; 0: skip")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy 10 times (reference for HBM traffic counters)")
    ap.add_argument("--kernel", choices=["append", "prefill", "prefill-f32", "decode-attn", "decode-attn-f32", "multistream",
                                         "multistream-attn", "decode-step", "decode-step-persistent"],
                    help="only run one hot-path kernel on synthetic inputs (short program for rocprofv3 passes)")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--kernel-len", type=int, default=4186,
                    help="attended positions of the decode-attn / decode-attn-f32 kernel modes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the KV-cache path would shard by "
              "KV head or by stream); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.kernel:
        kernel_only(args.kernel, args.kernel_reps, args.weights, args.kernel_len)
        return
    if args.copy_calibration:
        copy_calibration()
        return

    import dataclasses

    import qwenasr_amd as qa
    from qwenasr_amd import configs

    assert qa.device_count() > 0, "bench.py needs a HIP device"
    w = configs.CONFIGS[args.config]
    if args.kv_cache:
        w = dataclasses.replace(w, cache_type=qa.QA_CACHE_F16 if args.kv_cache == "f16" else qa.QA_CACHE_F32)
    kv_name = "f16" if w.cache_type == qa.QA_CACHE_F16 else "f32"
    plan = capacity_plan(w.prompt, args.warmup, args.steps, args.profile_steps,
                         args.bf16_steps if args.weights == "f32" else 0, args.persistent_steps)
    t0 = time.perf_counter()
    model = qa.Model(w.size, n_layers=w.n_layers, bf16=args.weights == "bf16-exact")
    x = qa.prompt_input(model, w.audio_tokens, w.prompt_tokens)
    log(f"synthetic {w.size.name} ({args.weights} weights) built in {time.perf_counter() - t0:.1f}s; "
        f"cache capacities {plan}")

    # ---- headline: batch-1 greedy decode of the config (every failure here ends the run: no line)
    dec, main_leg = decode_leg(qa, model, x, w.cache_type, plan["main"], args.warmup, args.steps, args.profile_steps)
    weights_streamed = "bf16 copies of bf16-exact weights" if dec.weights_bf16 else "f32"
    ctx0, dt = main_leg["ctx0"], main_leg["seconds"]
    log(f"prefill {w.prompt} positions: {main_leg['prefill_ms']:.1f} ms (first call "
        f"{main_leg['prefill_first_call_ms']:.1f} ms); device ms by family {main_leg['prefill_family_ms']}")
    log(f"timed {args.steps} decode steps at context {ctx0}..{ctx0 + args.steps} ({weights_streamed} weights "
        f"streamed): {dt * 1e3:.1f} ms ({main_leg['ms_per_step']:.4f} ms/token); per-step device ms by family "
        f"{main_leg['family_ms_per_step']}")
    elem = 2 if dec.weights_bf16 else 4
    wbytes = weight_bytes(model, elem)
    attn_us, L, attn_bytes, n_launch = attention_roofline(qa, dec, args.roofline_reps)
    dec.close()
    achieved = attn_bytes / (attn_us * 1e-6) / 1e9
    log(f"decode-step attention: {attn_us:.2f} us per launch pair over {n_launch} launches at L={L}: "
        f"{achieved:.0f} GB/s")
    traffic, traffic_note = measured_traffic(attn_bytes, kv_name)
    result = {
        "metric": METRIC,
        "value": round(args.steps / dt, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_leg["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": (f"synthetic (seeded N(0,0.02) weights{', rounded to bf16 values as in a converted bf16 checkpoint' if args.weights == 'bf16-exact' else ' streamed as f32'}, "
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
        "attn_us_per_layer": round(attn_us, 3),
        "prefill_ms": main_leg["prefill_ms"],
        "prefill_first_call_ms": main_leg["prefill_first_call_ms"],
        "prefill_family_ms": main_leg["prefill_family_ms"],
        "family_ms_per_step": main_leg["family_ms_per_step"],
        "weight_bytes_per_token": wbytes,
        "weight_stream_gbs": round(wbytes / (dt / args.steps) / 1e9, 1),
        "roofline_weights": (decode_weight_rooflines(model.cfg, elem, main_leg["family_ms_per_step"])
                             if main_leg["family_ms_per_step"] else None),
        "capacity_plan": plan,
    }

    # ---- secondary legs: each records its own error instead of ending the run
    def f32_cache():
        r = f32_cache_roofline(qa, model.cfg, L, max(2, args.roofline_reps // 2))
        log(f"f32-cache decode attention at L={r['attended_positions']}: {r['avg_launch_us']:.2f} us, "
            f"{r['achieved']:.0f} GB/s ({100 * r['frac']:.1f}% of peak)")
        return r

    def ms_roof():
        r = multistream_roofline(qa, model.cfg, max(2, args.roofline_reps // 4))
        log(f"config-4 multi-stream attention: {r['avg_launch_us']:.1f} us per layer, {r['achieved']:.0f} GB/s "
            f"({100 * r['frac']:.1f}% of peak)")
        return r

    def ms_roof4k():
        r = multistream_roofline(qa, model.cfg, max(2, args.roofline_reps // 4), lens=[4095] * 32,
                                 label="32 streams at 4k context")
        log(f"32 streams at 4k: {r['avg_launch_us']:.1f} us per layer, {r['achieved']:.0f} GB/s "
            f"({100 * r['frac']:.1f}% of peak)")
        return r

    def ms_decode():
        r = multistream_decode(qa, model, args.multistream_steps)
        log(f"config-4 decode, {r['streams']} streams: {r['ms_per_step']:.2f} ms per step, {r['tok_s']:.0f} tok/s "
            f"(device ms per step by family: {r['family_ms_per_step']})")
        return r

    def ms_decode_packed():
        # the opt-in packed f32 GEMMs (QA_GR_PACKED=1, read at decoder creation): q|k|v and o on weights reordered
        # for the f32 MFMA (the LM head is packed by default); another summation order than the default kernels
        os.environ["QA_GR_PACKED"] = "1"
        try:
            r = multistream_decode(qa, model, args.multistream_steps)
        finally:
            del os.environ["QA_GR_PACKED"]
        log(f"config-4 decode with the packed f32 GEMMs: {r['ms_per_step']:.2f} ms per step")
        return r

    guarded(result, "roofline_prefill_attn", lambda: prefill_attn_roofline(model.cfg, w.prompt, main_leg["prefill_family_ms"]))
    guarded(result, "roofline_f32_cache", f32_cache)
    guarded(result, "roofline_multistream", ms_roof)
    guarded(result, "roofline_multistream_4k", ms_roof4k)
    guarded(result, "multistream_decode", ms_decode)
    if args.weights == "f32":
        guarded(result, "multistream_decode_packed_f32", ms_decode_packed)
    def persistent_leg():
        # the same decode with every layer of a token in one persistent launch (LM head and pick separate)
        import numpy as np

        d = qa.Decoder(model, 1, plan["persistent"], w.cache_type)
        try:
            d.set_persistent(True)
            first = int(np.argmax(d.forward(x, 0)))
            ids = d.decode_streams(np.array([first], np.int32), args.warmup) if args.warmup else np.array([[first]], np.int32)
            got = ids[:, 0].tolist() if args.warmup else []
            qa.check(qa.lib.qa_device_synchronize())
            t0 = time.perf_counter()
            ids = d.decode_streams(np.array([int(ids[-1, 0])], np.int32), args.persistent_steps)
            qa.check(qa.lib.qa_device_synchronize())
            dt_p = time.perf_counter() - t0
            got += ids[:, 0].tolist()
        finally:
            d.close()
        n = min(len(got), len(main_leg["ids"]))
        r = {"steps": args.persistent_steps, "ms_per_step": round(dt_p * 1e3 / args.persistent_steps, 4),
             "tok_s": round(args.persistent_steps / dt_p, 3),
             "over_eager": round(dt_p / args.persistent_steps / (dt / args.steps), 3),
             "ids_equal_eager": got[:n] == main_leg["ids"][:n], "ids_compared": n,
             "mechanism": "one launch of 256 resident workgroups per token for all layers (grid "
                          "barriers between the six phases of a layer), then the LM head and the pick"}
        log(f"persistent decode step: {r['ms_per_step']:.4f} ms/token ({r['over_eager']:.2f}x the eager step), "
            f"ids equal to the eager run: {r['ids_equal_eager']} ({n} compared)")
        return r

    if args.persistent_steps > 0:
        guarded(result, "decode_persistent", persistent_leg)
    if args.no_cpu_baseline:
        result["cpu_baseline"] = None
    else:
        guarded(result, "cpu_baseline", lambda: cpu_baseline(model, ctx0, args.cpu_steps))

    if args.weights == "f32" and args.bf16_steps > 0:
        def bf16_leg():
            # the same draws rounded to bf16 values (in place: the f32 legs are done): the decoder streams
            # its bf16 copies, half the weight bytes, with f32 products and sums
            qa.check(qa.lib.qa_model_round_bf16(model.handle))
            x16 = qa.prompt_input(model, w.audio_tokens, w.prompt_tokens)   # prompt rows of the rounded table
            d16, leg = decode_leg(qa, model, x16, w.cache_type, plan["bf16_exact"], args.warmup, args.bf16_steps, 0)
            streamed = bool(d16.weights_bf16)
            d16.close()
            leg.pop("seconds")
            leg.pop("first_id")
            leg.pop("ids")
            leg["weights_streamed"] = "bf16 copies of bf16-exact weights" if streamed else "f32"
            leg["weight_bytes_per_token"] = weight_bytes(model, 2 if streamed else 4)
            log(f"bf16-exact weights: {leg['ms_per_step']:.4f} ms/token ({leg['tok_s']:.1f} tok/s), prefill "
                f"{leg['prefill_ms']:.1f} ms")
            if streamed and leg.get("prefill_family_ms"):
                leg["roofline_prefill_gemm"] = prefill_gemm_roofline(model.cfg, w.prompt, leg["prefill_family_ms"])
            r4 = multistream_decode(qa, model, max(4, args.multistream_steps // 2))
            leg["multistream_decode"] = r4
            log(f"bf16-exact weights, config-4 decode: {r4['ms_per_step']:.2f} ms per step")
            return leg

        guarded(result, "decode_bf16_exact_weights", bf16_leg)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
