"""Writes the golden fixtures of configs 0-4 from the CPU oracle (run once, on any x86-64 host).

    python tests/golden/make_golden.py [--configs 0,1,2,3,4] [--cfg4-streams 4] [--bf16]

Inputs come from the product's seeded generator (the same bits the GPU path receives); outputs come
from oracle/qa_oracle.c.  Each fixture records a checksum of its inputs so a drift of the generator
is caught before any comparison.  The reference's own goldens (real-weight JFK ids, README.md:301-303)
need a checkpoint and audio that do not exist here, so these fixtures are the oracle's.

--bf16 rounds the synthetic weights to bf16 values first (what a checkpoint converted from the released
bf16 weights holds, convert.py:386-387) and writes cfg{N}_bf16.json: the bench's own workload.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "qwenasr.cpp_amd"), os.path.join(ROOT, "oracle")]

import qa_oracle as orc  # noqa: E402
import qwenasr_amd as qa  # noqa: E402
from qwenasr_amd import configs  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


def write(name: str, obj: dict):
    path = os.path.join(OUT, name)
    with open(path, "w") as f:
        json.dump(obj, f, indent=1)
    print("wrote", path, flush=True)


def cfg0():
    w = configs.CONFIGS[0]
    model = qa.Model(w.size, n_layers=1)
    om = orc.OracleModel.from_product_model(model)
    x, k, v = configs.cfg0_inputs(model.cfg.hidden)
    cache = om.cache(w.max_seq, f16=False)
    cache.fill(k, v, 156)
    y = om.layer_forward_cached(0, x, 156, cache)
    write("cfg0.json", dict(config=0, input_digest=digest(x, k, v, model.tensor("text.blk.0.attn_q.weight")),
                            cur_len=cache.cur_len, y=y[0].tolist(), k_row=cache.k[0, :, 156].tolist(),
                            v_row=cache.v[0, :, 156].tolist()))


def greedy(index: int, bf16: bool = False):
    w = configs.CONFIGS[index]
    t0 = time.time()
    model = qa.Model(w.size, n_layers=w.n_layers, bf16=bf16)
    om = orc.OracleModel.from_product_model(model)
    x = qa.prompt_input(model, w.audio_tokens, w.prompt_tokens)
    cache = om.cache(w.max_seq, f16=w.cache_type == qa.QA_CACHE_F16)
    out = om.generate(x, w.new_tokens, qa.STOP_IDS, cache)
    assert out["rc"] == 0, out["rc"]
    write(f"cfg{index}{'_bf16' if bf16 else ''}.json",
          dict(config=index, input_digest=digest(x, model.tensor("text.blk.0.attn_q.weight")), bf16_weights=bf16,
                                   prompt_tokens=w.prompt, requested=w.new_tokens, ids=out["ids"],
                                   stopped=out["stopped"], total_tokens=out["total_tokens"], cur_len=out["cur_len"],
                                   margins=out["margins"], runner_up=out["runner_up"],
                                   oracle_seconds=round(time.time() - t0, 1)))


def cfg4(n_check: int, bf16: bool = False):
    w = configs.CONFIGS[4]
    t0 = time.time()
    model = qa.Model(w.size, n_layers=w.n_layers, bf16=bf16)
    om = orc.OracleModel.from_product_model(model)
    lens = configs.cfg4_lengths(w.streams)
    first = configs.cfg4_first_ids(w.streams)
    order = np.argsort(lens)
    pick = sorted({int(order[0]), int(order[-1])} | {int(s) for s in order[np.linspace(1, w.streams - 2, max(n_check - 2, 0)).astype(int)]})
    streams = {}
    for s in pick:
        L = int(lens[s])
        k, v = configs.cfg4_stream_kv(s, L)
        cache = om.cache(L + w.steps, f16=True)
        cache.fill(k, v, L)
        del k, v
        ids, marg, second = om.decode_steps(cache, int(first[s]), w.steps)
        streams[str(s)] = dict(length=L, first_id=int(first[s]), ids=ids, margins=marg, runner_up=second,
                               cur_len=cache.cur_len)
        print(f"  cfg4 stream {s} (len {L}) done at {time.time() - t0:.0f}s", flush=True)
    write(f"cfg4{'_bf16' if bf16 else ''}.json", dict(config=4, bf16_weights=bf16, lengths=lens.tolist(), first_ids=first.tolist(), steps=w.steps,
                            streams=streams, oracle_seconds=round(time.time() - t0, 1)))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--configs", default="0,1,2,3,4")
    ap.add_argument("--cfg4-streams", type=int, default=4)
    ap.add_argument("--bf16", action="store_true", help="bf16-exact weights (configs 1-4)")
    args = ap.parse_args()
    for c in [int(v) for v in args.configs.split(",")]:
        t = time.time()
        if c == 0:
            cfg0()
        elif c == 4:
            cfg4(args.cfg4_streams, bf16=args.bf16)
        elif args.bf16:
            greedy(c, bf16=True)
        else:
            greedy(c)
        print(f"config {c}: {time.time() - t:.1f}s", flush=True)


if __name__ == "__main__":
    main()
